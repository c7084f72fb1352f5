// quant_host.cpp - host side of the MXFP8 quantisers: the C ABI of include/mxfp8_quant.h.
//
// Argument checks, then launches of the kernels of quant_kernels.hip (embedded at build time, loaded once per
// device). No call allocates device memory; the V tensor scale keeps its partial maxima in the caller's descale buffer.

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>

#include "../../include/mxfp8_quant.h"
#include "module_cache.h"

#ifndef MXQ_HSACO_PATH
#error "MXQ_HSACO_PATH must name the gfx950 code object built from quant_kernels.hip"
#endif
asm(".section .rodata.mxq_hsaco,\"a\",@progbits\n"
    ".balign 4096\n"
    ".global mxfp8_quant_hsaco_begin\n"
    "mxfp8_quant_hsaco_begin:\n"
    ".incbin \"" MXQ_HSACO_PATH "\"\n"
    ".global mxfp8_quant_hsaco_end\n"
    "mxfp8_quant_hsaco_end:\n"
    ".previous\n");
extern "C" const unsigned char mxfp8_quant_hsaco_begin[];
extern "C" const unsigned char mxfp8_quant_hsaco_end[];

namespace {

using fmha_internal::fail;

// The kernels' by-value argument structs (quant_kernels.hip).
struct QuantRowsArgs {
    const void* x;
    void* q;
    void* scale;
    uint64_t rows;
    float mul;
    uint32_t pad;
};
struct QuantTensorArgs {
    const void* x;
    void* q;
    void* descale;
    uint64_t n;
};
struct QuantSeq32Args {
    const void* x;
    void* q;
    void* scale;
    uint32_t B, SK, HK, nblk;
};
static_assert(sizeof(QuantRowsArgs) == 40, "rows kernarg");
static_assert(sizeof(QuantTensorArgs) == 32, "tensor kernarg");
static_assert(sizeof(QuantSeq32Args) == 40, "seq32 kernarg");

const char* const kQuantNames[4] = {
    "fmha_mxfp8_quant_rows", "fmha_mxfp8_quant_amax", "fmha_mxfp8_quant_tensor", "fmha_mxfp8_quant_seq32",
};
enum { Q_ROWS = 0, Q_AMAX = 1, Q_TENSOR = 2, Q_SEQ32 = 3 };
// quant_kernels.hip: the amax pass runs exactly 512 workgroups and leaves one partial maximum each in descale words
// [512, 1024); the descale buffer therefore spans 4096 bytes, the size the FMHA requires of it anyway.
constexpr uint32_t kAmaxGroups = 512;
constexpr uint64_t kDescaleBytes = 4096;

fmha_internal::ModuleCache<4> g_quant(mxfp8_quant_hsaco_begin, mxfp8_quant_hsaco_end, kQuantNames);

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

// Workgroups of the quantising pass over `chunks` 8-element chunks: enough to cover the chunks once, at most 4 per CU
// of a 256-CU part (each workgroup first reduces the 512 partial maxima, so fewer, longer workgroups read less).
uint32_t stride_grid(uint64_t chunks) {
    const uint64_t g = (chunks + 255) / 256;
    return (uint32_t)(g < 1 ? 1 : g > 1024 ? 1024 : g);
}

}  // namespace

extern "C" {

int fmha_mxfp8_quantize_rows(const void* x, void* q, void* scale, int64_t rows, float mul, uint64_t bytes_x, uint64_t bytes_q,
                             uint64_t bytes_scale, void* stream, char* err, size_t errlen) {
    if (rows < 1 || rows > (int64_t)0xFFFFFFFF * 64) return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "rows outside [1, 2^38)");
    if (!x || !q || !scale) return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "null pointer");
    if (!aligned(x, 16) || !aligned(q, 8) || !aligned(scale, 4))
        return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "x needs 16-byte, q 8-byte and scale 4-byte alignment");
    const uint64_t r = (uint64_t)rows;
    if (bytes_x < r * 256) return fail(err, errlen, FMHA_ERR_EXTENT, "GV-HOST-EXTENT", "x: buffer smaller than rows * 256 bytes");
    if (bytes_q < r * 128) return fail(err, errlen, FMHA_ERR_EXTENT, "GV-HOST-EXTENT", "q: buffer smaller than rows * 128 bytes");
    if (bytes_scale < r * 4) return fail(err, errlen, FMHA_ERR_EXTENT, "GV-HOST-EXTENT", "scale: buffer smaller than rows * 4 bytes");
    QuantRowsArgs a = {x, q, scale, r, mul, 0u};
    return g_quant.launch(Q_ROWS, &a, sizeof(a), (uint32_t)((r + 63) / 64), 1, 1, 256, stream, err, errlen);   // 64 rows per workgroup
}

int fmha_mxfp8_quantize_tensor(const void* x, void* q, void* descale, int64_t n, uint64_t bytes_x, uint64_t bytes_q,
                               uint64_t bytes_descale, void* stream, char* err, size_t errlen) {
    if (n < 8 || n % 8 != 0) return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "n must be a positive multiple of 8");
    if (!x || !q || !descale) return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "null pointer");
    if (!aligned(x, 16) || !aligned(q, 8) || !aligned(descale, 4))
        return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "x needs 16-byte, q 8-byte and descale 4-byte alignment");
    const uint64_t un = (uint64_t)n;
    if (bytes_x < un * 2) return fail(err, errlen, FMHA_ERR_EXTENT, "GV-HOST-EXTENT", "x: buffer smaller than n * 2 bytes");
    if (bytes_q < un) return fail(err, errlen, FMHA_ERR_EXTENT, "GV-HOST-EXTENT", "q: buffer smaller than n bytes");
    if (bytes_descale < kDescaleBytes) return fail(err, errlen, FMHA_ERR_EXTENT, "GV-HOST-EXTENT", "descale: buffer smaller than 4096 bytes");
    QuantTensorArgs a = {x, q, descale, un};
    int rc = g_quant.launch(Q_AMAX, &a, sizeof(a), kAmaxGroups, 1, 1, 256, stream, err, errlen);
    if (rc == FMHA_OK) rc = g_quant.launch(Q_TENSOR, &a, sizeof(a), stride_grid(un / 8), 1, 1, 256, stream, err, errlen);
    return rc;
}

size_t fmha_mxfp8_seq32_scale_bytes(int64_t B, int64_t SK, int64_t HK) {
    if (B < 1 || SK < 1 || HK < 1) return 0;
    return (size_t)((uint64_t)B * (uint64_t)((SK + 31) / 32) * (uint64_t)HK * 128u);
}

int fmha_mxfp8_quantize_seq32(const void* x, void* q, void* scale, int32_t B, int32_t SK, int32_t HK, uint64_t bytes_x,
                              uint64_t bytes_q, uint64_t bytes_scale, void* stream, char* err, size_t errlen) {
    if (B < 1 || SK < 1 || HK < 1) return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "B, SK, HK must be >= 1");
    if (!x || !q || !scale) return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "null pointer");
    if (!aligned(x, 16) || !aligned(q, 8) || !aligned(scale, 8))
        return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "x needs 16-byte, q and scale 8-byte alignment");
    const uint64_t elems = (uint64_t)B * (uint64_t)SK * (uint64_t)HK * 128u;
    const uint32_t nblk = (uint32_t)((SK + 31) / 32);
    if (bytes_x < elems * 2) return fail(err, errlen, FMHA_ERR_EXTENT, "GV-HOST-EXTENT", "x: buffer smaller than B*SK*HK*256 bytes");
    if (bytes_q < elems) return fail(err, errlen, FMHA_ERR_EXTENT, "GV-HOST-EXTENT", "q: buffer smaller than B*SK*HK*128 bytes");
    if (bytes_scale < fmha_mxfp8_seq32_scale_bytes(B, SK, HK))
        return fail(err, errlen, FMHA_ERR_EXTENT, "GV-HOST-EXTENT", "scale: buffer smaller than B*ceil(SK/32)*HK*128 bytes");
    const uint64_t lanes = (uint64_t)B * nblk * (uint64_t)HK * 16u;
    if ((lanes + 255) / 256 > 0xFFFFFFFFull) return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "tensor too large");
    QuantSeq32Args a = {x, q, scale, (uint32_t)B, (uint32_t)SK, (uint32_t)HK, nblk};
    return g_quant.launch(Q_SEQ32, &a, sizeof(a), (uint32_t)((lanes + 255) / 256), 1, 1, 256, stream, err, errlen);
}

}  // extern "C"
