/*
 * q38a measurement probes: the ceilings this GPU reaches, measured beside the published peaks
 * (MI355X: 8 TB/s HBM, 2.5 PFLOP/s dense fp16/bf16 MFMA). No counterpart in the reference; used by
 * bench.py for the roofline's measured peaks. Both launch asynchronously on `stream`.
 */
#ifndef Q38A_PROBE_H
#define Q38A_PROBE_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* MFMA issue ceiling: `iters` rounds of eight independent v_mfma_f32_32x32x16_f16 per wave, two
 * four-wave workgroups per CU, no memory traffic. *flops = the launch's dense fp16 flops.
 * sink: device floats, one per workgroup (2 x CUs), written only to keep the work live. */
int q38a_probe_mfma(float* sink, int iters, void* stream, double* flops);

/* HBM read ceiling: reads `bytes` (a multiple of 16) of device memory once with 16-byte loads;
 * sink: sink_len device floats, also the number of 256-thread workgroups. */
int q38a_probe_read(const void* buf, size_t bytes, float* sink, int sink_len, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* Q38A_PROBE_H */
