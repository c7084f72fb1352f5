// MXFP8 quantisers that produce the FMHA's inputs from bf16 tensors on the GPU (gfx950).
//
// The rule is the one the reference's own input generator applies (tests/gpu/ref_host.cpp:224-251):
//   * Q and K rows: per 32-element block along head_dim, E8M0 = clamp(floor(log2 amax) - 8 + 127, 0, 254), elements
//     e4m3 (OCP E4M3FN) of x * 2^(127 - E8M0), round to nearest even, saturating at +-448 (NaN -> +448, as the
//     generator's `!(a < 448)` test does). Q is pre-multiplied by `mul` (log2(e)/sqrt(128) for the reference's
//     softmax convention) in f32 before the block maximum is taken.
//   * V, reference layout: one f32 descale d = amax / 448 for the whole tensor, elements e4m3(x / d) (IEEE division).
//   * V, sequence-blocked layout (an extension): per 32 keys along the sequence and per head_dim column, the Q/K rule.
// The reference's GEMM-side quantiser family (crates/amdgpu-kernels/src/rows/mxquant.rs) uses a different scale
// rule and layout; these kernels follow the FMHA generator so their bytes are the FMHA's inputs bit for bit.
//
// All three are HBM-bound streaming kernels: every lane moves 16-byte bf16 chunks (8 elements) in and 8-byte e4m3
// chunks out; a 32-element block lives in 4 adjacent lanes (rows) or in one lane (sequence blocks).
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// An 8-byte vector store written through the L2 (sc0 sc1), so that no dirty lines are left for the kernel-end write-back.
__device__ inline void store8_system(void* ptr, u32x2 x) {
    asm volatile("global_store_dwordx2 %0, %1, off sc0 sc1\n\ts_nop 1" ::"v"(ptr), "v"(x) : "memory");
}

__device__ inline float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ inline float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// E8M0 byte of a block maximum: floor(log2 amax) - 8 + 127 clamped to [0, 254]. For a normal amax the floor of
// log2 is the unbiased exponent, so the byte is the biased exponent field minus 8; zero and subnormal maxima
// (floor(log2) <= -127) clamp to 0.
__device__ inline uint32_t e8m0_of_amax(float amax) {
    const uint32_t ef = (__float_as_uint(amax) >> 23) & 0xffu;
    return ef > 8u ? ef - 8u : 0u;
}

// 2^(127 - e) as an f32 (e in [0, 253]: the exponent field 254 - e is a normal exponent).
__device__ inline float inv_scale(uint32_t e) { return __uint_as_float((254u - e) << 23); }

// (x * s) + 0, the product rounded on its own first (the build keeps the two operations apart: -ffp-contract=off).
// The generator rounds x * 2^(127 - E8M0) to f32 and takes the sign byte from `f < 0` (ref_host.cpp:219), so a
// product that rounds to -0 must encode as +0; the hardware conversion would keep the sign of -0. Adding +0 to the
// rounded product maps -0 to +0 and changes nothing else (a fused multiply-add would round the exact negative
// product to -0 and keep it).
__device__ inline float scaled(float x, float s) { return x * s + 0.0f; }

// The generator's saturation: |x| >= 448 goes to +-448 and NaN to +448 (its sign byte is `x < 0`). fminf returns
// the non-NaN operand, so NaN becomes 448 in the first step.
__device__ inline float sat448(float x) { return fmaxf(fminf(x, 448.0f), -448.0f); }

// Four f32 (already in range) -> one word of four e4m3 bytes, element 0 in the low byte. The conversion rounds to
// nearest even (the MODE register's default round mode).
__device__ inline uint32_t pack4_e4m3(float a, float b, float c, float d) {
    int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
    return (uint32_t)w;
}

// Max over the 4 lanes of a quad (one 32-element block) by two quad_perm DPP moves.
__device__ inline float quad_max(float v) {
    float o = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xb1, 0xf, 0xf, false));  // [1,0,3,2]
    v = fmaxf(v, o);
    o = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4e, 0xf, 0xf, false));        // [2,3,0,1]
    return fmaxf(v, o);
}

}  // namespace

// Kernel arguments (plain structs passed by value; the host fills the same layouts).
struct QuantRowsArgs {
    const uint16_t* x;   // [rows, 128] bf16
    uint8_t* q;          // [rows, 128] e4m3
    uint8_t* scale;      // [rows, 4] E8M0
    uint64_t rows;
    float mul;
    uint32_t pad;
};

struct QuantTensorArgs {
    const uint16_t* x;   // [n] bf16, n % 8 == 0
    uint8_t* q;          // [n] e4m3
    float* descale;      // 1024 f32: [0] the descale; [kQuantPartial, +kQuantAmaxGroups) the amax pass's partials
    uint64_t n;
};
// The amax pass runs exactly this many workgroups (the host launches it so), one partial maximum each.
constexpr uint32_t kQuantAmaxGroups = 512;
constexpr uint32_t kQuantPartial = 512;

struct QuantSeq32Args {
    const uint16_t* x;   // [B, SK, HK, 128] bf16
    uint8_t* q;          // [B, SK, HK, 128] e4m3
    uint8_t* scale;      // [B, ceil(SK/32), HK, 128] E8M0
    uint32_t B, SK, HK, nblk;
};

// Rows: 16 lanes per 128-element row (8 elements per lane), 4 lanes per 32-element block. A workgroup covers
// kRowsPerGroup rows: each 16-lane group takes 4 rows 16 apart and issues their four 16-byte loads before using any
// (64 bytes in flight per lane). Lane 0 of a row writes the row's 4 scale bytes as one word.
constexpr uint32_t kRowsPerGroup = 64;

extern "C" __global__ void __launch_bounds__(256) fmha_mxfp8_quant_rows(QuantRowsArgs a) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t c = threadIdx.x & 15u;   // 8-element chunk of the row
    const uint64_t row0 = (uint64_t)blockIdx.x * kRowsPerGroup + (threadIdx.x >> 4);
    u32x4 w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint64_t row = row0 + 16u * j;
        const uint64_t r = row < a.rows ? row : 0;   // rows past the end (the last workgroup) read row 0, store nothing
        w[j] = *reinterpret_cast<const u32x4*>(a.x + r * 128u + c * 8u);
    }
    const uint32_t base = lane & ~15u;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint64_t row = row0 + 16u * j;
        float v[8];
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = bf16_lo(w[j][i]) * a.mul;
            v[2 * i + 1] = bf16_hi(w[j][i]) * a.mul;
        }
        float m = 0.0f;
        for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(v[i]));   // fmaxf drops NaN, as std::max(amax, NaN) keeps amax
        m = quad_max(m);
        const uint32_t e = e8m0_of_amax(m);
        const float s = inv_scale(e);
        u32x2 out;
        out[0] = pack4_e4m3(sat448(scaled(v[0], s)), sat448(scaled(v[1], s)), sat448(scaled(v[2], s)), sat448(scaled(v[3], s)));
        out[1] = pack4_e4m3(sat448(scaled(v[4], s)), sat448(scaled(v[5], s)), sat448(scaled(v[6], s)), sat448(scaled(v[7], s)));
        // the row's four block bytes sit in lanes c = 0, 4, 8, 12 of its 16-lane group
        const uint32_t e1 = __shfl(e, base + 4, 64), e2 = __shfl(e, base + 8, 64), e3 = __shfl(e, base + 12, 64);
        if (row < a.rows) {
            store8_system(a.q + row * 128u + c * 8u, out);
            if (c == 0) *reinterpret_cast<uint32_t*>(a.scale + row * 4u) = e | (e1 << 8) | (e2 << 16) | (e3 << 24);
        }
    }
}

// Tensor scale, pass 1: kQuantAmaxGroups workgroups stride over the tensor; workgroup g stores its maximum |x| into
// descale[kQuantPartial + g] (plain stores: every slot is rewritten by every call, so nothing needs clearing and no
// two workgroups touch one address). NaN elements are skipped (fmaxf), as std::max skips them in the generator's
// running maximum.
extern "C" __global__ void __launch_bounds__(256) fmha_mxfp8_quant_amax(QuantTensorArgs a) {
    __shared__ float part[4];
    const uint64_t nchunk = a.n / 8u;
    const uint64_t stride = (uint64_t)gridDim.x * 256u;
    float m = 0.0f;
    uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    for (; i + 3 * stride < nchunk; i += 4 * stride) {   // four 16-byte loads in flight per lane
        u32x4 w[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) w[u] = *reinterpret_cast<const u32x4*>(a.x + (i + u * stride) * 8u);
#pragma unroll
        for (int u = 0; u < 4; ++u)
            for (int j = 0; j < 4; ++j) m = fmaxf(m, fmaxf(fabsf(bf16_lo(w[u][j])), fabsf(bf16_hi(w[u][j]))));
    }
    for (; i < nchunk; i += stride) {
        const u32x4 w = *reinterpret_cast<const u32x4*>(a.x + i * 8u);
        for (int j = 0; j < 4; ++j) m = fmaxf(m, fmaxf(fabsf(bf16_lo(w[j])), fabsf(bf16_hi(w[j]))));
    }
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if ((threadIdx.x & 63u) == 0) part[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) a.descale[kQuantPartial + blockIdx.x] = fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3]));
}

// Tensor scale, pass 2: every workgroup reduces the kQuantAmaxGroups partial maxima, then d = amax / 448 and
// q = e4m3(x / d), both divisions correctly rounded as the generator's double divisions rounded to f32 are.
// Workgroup 0 writes d to descale[0].
//
// x / d is computed as q1 = q0 + (x - q0 d) r with r = RN(1/d), q0 = RN(x r) and the remainder from one fused
// multiply-add, which is the correctly rounded quotient (Markstein's theorem: r within half an ulp of 1/d, q0 within
// one ulp of x/d, remainder exact) as long as nothing leaves the normal range. The lanes with d, x or q0 outside
// [2^-96, 2^96] take the full division instead (zero x stays on the fast path: it yields +-0 either way). Checked
// against the correctly rounded division for every bf16 x over 40000 divisors, all-ones and power-of-two
// mantissas included.
// The fast quotient of x / d, and whether it is valid (`ok` is cleared when x or the quotient is out of range).
__device__ inline float div_fast(float x, float d, float r, bool& ok) {
    const float q0 = x * r;
    ok = ok && ((fabsf(x) >= 0x1p-96f && fabsf(q0) >= 0x1p-96f) || x == 0.0f);
    return __builtin_fmaf(__builtin_fmaf(-q0, d, x), r, q0);
}

extern "C" __global__ void __launch_bounds__(256) fmha_mxfp8_quant_tensor(QuantTensorArgs a) {
    __shared__ float part[4];
    float m = 0.0f;
    for (uint32_t i = threadIdx.x; i < kQuantAmaxGroups; i += 256u) m = fmaxf(m, a.descale[kQuantPartial + i]);
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if ((threadIdx.x & 63u) == 0) part[threadIdx.x >> 6] = m;
    __syncthreads();
    const float amax = fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3]));
    const float d = __fdiv_rn(amax, 448.0f);
    const float r = __fdiv_rn(1.0f, d);
    const bool dfast = d >= 0x1p-96f && d <= 0x1p96f;
    const uint64_t nchunk = a.n / 8u;
    const uint64_t stride = (uint64_t)gridDim.x * 256u;
    // four chunks per pass, their loads issued together (chunks past the end read chunk 0 and store nothing)
    for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < nchunk; i += 4 * stride) {
        u32x4 w[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint64_t c = i + u * stride;
            w[u] = *reinterpret_cast<const u32x4*>(a.x + (c < nchunk ? c : 0) * 8u);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            float y[8];
            bool ok = dfast;
            for (int j = 0; j < 4; ++j) {
                y[2 * j] = div_fast(bf16_lo(w[u][j]), d, r, ok);
                y[2 * j + 1] = div_fast(bf16_hi(w[u][j]), d, r, ok);
            }
            if (!ok) {   // rare: one out-of-range element sends its whole chunk through the full division
                for (int j = 0; j < 4; ++j) {
                    y[2 * j] = __fdiv_rn(bf16_lo(w[u][j]), d);
                    y[2 * j + 1] = __fdiv_rn(bf16_hi(w[u][j]), d);
                }
            }
            for (int j = 0; j < 8; ++j) y[j] = sat448(y[j] + 0.0f);   // +0: -0 -> +0 (see scaled)
            u32x2 out;
            out[0] = pack4_e4m3(y[0], y[1], y[2], y[3]);
            out[1] = pack4_e4m3(y[4], y[5], y[6], y[7]);
            const uint64_t c = i + u * stride;
            if (c < nchunk) store8_system(a.q + c * 8u, out);
        }
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) a.descale[0] = d;
}

// Sequence blocks: one lane per (b, 32-key block, kv head, 8-column chunk). Pass 1 takes the lane's 8 column maxima
// over the block's keys, pass 2 reads the same 32 chunks again (from L2) and writes their e4m3 bytes, then the lane
// writes its 8 scale bytes. A ragged last block (SK % 32 != 0) takes its maxima over the keys that exist.
extern "C" __global__ void __launch_bounds__(256) fmha_mxfp8_quant_seq32(QuantSeq32Args a) {
    const uint64_t gid = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    const uint32_t c = (uint32_t)(gid & 15u);
    uint64_t t = gid >> 4;
    const uint32_t hk = (uint32_t)(t % a.HK);
    t /= a.HK;
    const uint32_t blk = (uint32_t)(t % a.nblk);
    const uint64_t b = t / a.nblk;
    if (b >= a.B) return;
    const uint32_t k0 = blk * 32u;
    const uint32_t nk = min(32u, a.SK - k0);
    const uint64_t row_stride = (uint64_t)a.HK * 128u;
    const uint64_t base = ((uint64_t)b * a.SK + k0) * row_stride + (uint64_t)hk * 128u + c * 8u;
    float m[8];
    for (int j = 0; j < 8; ++j) m[j] = 0.0f;
    for (uint32_t k = 0; k < nk; ++k) {
        const u32x4 w = *reinterpret_cast<const u32x4*>(a.x + base + k * row_stride);
        for (int j = 0; j < 4; ++j) {
            m[2 * j] = fmaxf(m[2 * j], fabsf(bf16_lo(w[j])));
            m[2 * j + 1] = fmaxf(m[2 * j + 1], fabsf(bf16_hi(w[j])));
        }
    }
    uint32_t e[8];
    float s[8];
    for (int j = 0; j < 8; ++j) {
        e[j] = e8m0_of_amax(m[j]);
        s[j] = inv_scale(e[j]);
    }
    for (uint32_t k = 0; k < nk; ++k) {
        const u32x4 w = *reinterpret_cast<const u32x4*>(a.x + base + k * row_stride);
        u32x2 out;
        out[0] = pack4_e4m3(sat448(scaled(bf16_lo(w[0]), s[0])), sat448(scaled(bf16_hi(w[0]), s[1])),
                            sat448(scaled(bf16_lo(w[1]), s[2])), sat448(scaled(bf16_hi(w[1]), s[3])));
        out[1] = pack4_e4m3(sat448(scaled(bf16_lo(w[2]), s[4])), sat448(scaled(bf16_hi(w[2]), s[5])),
                            sat448(scaled(bf16_lo(w[3]), s[6])), sat448(scaled(bf16_hi(w[3]), s[7])));
        *reinterpret_cast<u32x2*>(a.q + base + k * row_stride) = out;
    }
    u32x2 sc;
    sc[0] = e[0] | (e[1] << 8) | (e[2] << 16) | (e[3] << 24);
    sc[1] = e[4] | (e[5] << 8) | (e[6] << 16) | (e[7] << 24);
    *reinterpret_cast<u32x2*>(a.scale + (((uint64_t)b * a.nblk + blk) * a.HK + hk) * 128u + c * 8u) = sc;
}
