/*
 * rrr_probe.h -- platform probes of librrr_hip.so, used by the benchmark to
 * report what the device itself reaches next to what the decode-path kernels
 * reach.  They have no counterpart in the reference (its benchmark reports
 * only end-to-end timings).  Same conventions as rrr_hip.h: int status,
 * arguments checked before any HIP call, asynchronous when the context is.
 */
#ifndef RRR_PROBE_H
#define RRR_PROBE_H

#include "rrr_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Streaming read of the first `bytes` (a multiple of 16) of `buf`: every
 * 16-byte unit is loaded once (non-temporal, 4 workgroups of 1024 threads per
 * CU); nothing is written except, under a condition no input meets, the
 * 4-byte `sink`.  bytes / time is the HBM read rate one launch of that size
 * reaches; a read of twice the Infinity Cache's 256 MB evicts it. */
int rrr_probe_read(rrr_ctx *ctx, const rrr_buf *buf, uint64_t bytes, rrr_buf *sink);

/* Per-launch read floor of a GEMV's byte count: one workgroup of 1024
 * threads per CU reads a contiguous share of ceil(bytes / CUs) bytes (rounded
 * up to 16 KB), every lane issuing all of its 16-byte non-temporal loads
 * (at most 16) before using any.  bytes a positive multiple of 16, at most
 * CUs * 256 KB (RRR_ERR_UNSUPPORTED beyond).  bytes / time is what one launch
 * that only reads those bytes, spread over every CU as the GEMVs spread their
 * rows, reaches. */
int rrr_probe_read_shares(rrr_ctx *ctx, const rrr_buf *buf, uint64_t bytes, rrr_buf *sink);

/* Phase timestamps of one batch-1 K-quant GEMV launch: the launch the named
 * entry point makes for these arguments (op RRR_PHASES_PLAIN = rrr_gemv with
 * M = 1, _RMSNORM = rrr_gemv_rmsnorm, _RESIDUAL = rrr_gemv_residual with
 * act_kind / act_param, _RMSNORM_SILU = rrr_gemv_rmsnorm_silu with N = F),
 * the same kernel instantiated to read the 100 MHz constant clock at its
 * phases.  Outputs are those of the entry point.  stamps: at least
 * CUs * 16 * 16 * 8 bytes; wave w of workgroup b writes 16 u64 at
 * (b * waves + w) * 16: 0 start, 1 activations landed, 2 after the fused
 * RMSNorm scale, 3 activations encoded, 4 / 6 the first tile's super-block
 * 0 / 1 staged and 5 / 7 multiplied, 8-11 the same for the last tile, 12 the
 * wave's row partials written, 13 past the final workgroup barrier, 14 end
 * (its stores complete); 0 where a phase does not occur.  *grid_out and
 * *waves_out give the launch shape. */
enum { RRR_PHASES_PLAIN = 0, RRR_PHASES_RMSNORM = 1, RRR_PHASES_RESIDUAL = 2, RRR_PHASES_RMSNORM_SILU = 3 };
int rrr_probe_gemv_phases(rrr_ctx *ctx, uint32_t op, uint32_t act_kind, uint32_t act_param, const rrr_buf *x,
                          const rrr_buf *gamma, float eps, const rrr_buf *W, uint32_t type, rrr_buf *y, uint32_t K,
                          uint32_t N, rrr_buf *stamps, uint32_t *grid_out, uint32_t *waves_out);

/* Matrix-core rate: `waves_per_cu` waves on every CU (a multiple of 4, at most
 * 32) each run `iters` rounds of 4 independent MFMAs of `kind`.  Operations per
 * launch = CUs * waves_per_cu * iters * 4 * ops_per_mfma, ops_per_mfma
 * = 2*16*16*32 (16x16x32 f16), 2*32*32*16 (32x32x16 f16), 2*16*16*64
 * (16x16x64 int8). */
enum { RRR_PROBE_MFMA_F16_16X16X32 = 0, RRR_PROBE_MFMA_F16_32X32X16 = 1, RRR_PROBE_MFMA_I8_16X16X64 = 2 };
int rrr_probe_mfma(rrr_ctx *ctx, uint32_t kind, uint32_t waves_per_cu, uint32_t iters, rrr_buf *sink);
/* CUs of the context's device (the probes' grid unit); 0 without a device. */
uint32_t rrr_probe_cus(rrr_ctx *ctx);

#ifdef __cplusplus
}
#endif

#endif /* RRR_PROBE_H */
