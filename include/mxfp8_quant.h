/* mxfp8_quant.h - C ABI of the on-GPU MXFP8 quantisers that produce the FMHA's inputs (gfx950).
 *
 * The reference has no quantiser for this path: its inputs come from the host generator of
 * tests/gpu/ref_host.cpp:224-251 (REF_DATA=normal), and its GEMM-side quantiser family
 * (crates/amdgpu-kernels/src/rows/mxquant.rs, ABI x @0, q @8, scale @16, M @24) emits other layouts.
 * These entry points apply the generator's rule on the GPU, so their bytes are the FMHA's Q/K/V/scale
 * inputs exactly as the reference's generator would write them for the same (bf16) values:
 *   - rows (Q, K): per 32-element block along head_dim, E8M0 = clamp(floor(log2 amax) - 8 + 127, 0, 254);
 *     elements e4m3 of x * 2^(127 - E8M0), round to nearest even, saturating at +-448 (ref_host.cpp:239-247);
 *   - tensor (V): one f32 descale d = amax / 448, elements e4m3(x / d) (ref_host.cpp:248-251);
 *   - seq32 (V, extension): per 32 keys along the sequence and per head_dim column, the rows rule.
 * Inputs are bf16; `mul` multiplies the input in f32 before the block maximum (the caller's softmax fold:
 * log2(e)/sqrt(128) for Q, 1 for K). NaN inputs quantise to +448 as in the generator; +-Inf inputs are
 * outside the generator's domain (the block then takes E8M0 247).
 *
 * All pointers are device pointers; every call is asynchronous on `stream` (a hipStream_t, NULL = the
 * null stream), allocates nothing and returns FMHA_OK or an FMHA_ERR_* code of fmha_mxfp8.h with a
 * "GV-HOST-..." message in `err` (may be NULL).
 */
#ifndef MXFP8_QUANT_H
#define MXFP8_QUANT_H

#include <stddef.h>
#include <stdint.h>

#include "fmha_mxfp8.h"

#ifdef __cplusplus
extern "C" {
#endif

/* x [rows, 128] bf16 (16-byte aligned) -> q [rows, 128] e4m3 (8-byte aligned), scale [rows, 4] E8M0
 * (4-byte aligned). For the FMHA, rows = B*S*H (Q) or B*SK*HK (K); the FMHA also needs the zeroed slack
 * behind the scales (fmha_mxfp8.h), which this call neither writes nor needs. */
int fmha_mxfp8_quantize_rows(const void* x, void* q, void* scale, int64_t rows, float mul,
                             uint64_t bytes_x, uint64_t bytes_q, uint64_t bytes_scale,
                             void* stream, char* err, size_t errlen);

/* x [n] bf16 (n % 8 == 0, 16-byte aligned) -> q [n] e4m3, descale[0] = amax / 448 (f32).
 * `descale` is the FMHA's V-descale buffer (bytes_descale >= 4096, as fmha_mxfp8.h requires of it): between the
 * call's two launches, f32 words [512, 1024) hold per-workgroup partial maxima (rewritten by every call). */
int fmha_mxfp8_quantize_tensor(const void* x, void* q, void* descale, int64_t n,
                               uint64_t bytes_x, uint64_t bytes_q, uint64_t bytes_descale,
                               void* stream, char* err, size_t errlen);

/* x [B, SK, HK, 128] bf16 -> q [B, SK, HK, 128] e4m3, scale [B, ceil(SK/32), HK, 128] E8M0 (8-byte aligned). */
int fmha_mxfp8_quantize_seq32(const void* x, void* q, void* scale, int32_t B, int32_t SK, int32_t HK,
                              uint64_t bytes_x, uint64_t bytes_q, uint64_t bytes_scale,
                              void* stream, char* err, size_t errlen);

/* Bytes of the seq32 scale tensor: B * ceil(SK/32) * HK * 128. */
size_t fmha_mxfp8_seq32_scale_bytes(int64_t B, int64_t SK, int64_t HK);

#ifdef __cplusplus
}
#endif
#endif /* MXFP8_QUANT_H */
