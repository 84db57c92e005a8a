// Causal chunked prefill attention (placeholder until the MFMA kernel lands).
#include "plan.hpp"

namespace q38a {

int launch_attention_prefill(const q38a_attention_params&, const q38a_batch_desc&, const q38a_kv_cache_desc&,
                             hipStream_t) {
  return set_error(Q38A_ERR_UNSUPPORTED, "attention_prefill: not built yet");
}

int launch_attention_ragged(const q38a_attention_params&, const q38a_batch_desc&, const q38a_kv_cache_desc&,
                            hipStream_t) {
  return set_error(Q38A_ERR_UNSUPPORTED, "attention_ragged: not built yet");
}

}  // namespace q38a
