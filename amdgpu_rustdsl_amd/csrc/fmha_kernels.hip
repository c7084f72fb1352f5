// fmha_kernels.hip - MXFP8 FMHA forward, head dim 128, hand-written HIP for gfx950 (MI355X).
//
// Four kernels with the reference's names and kernarg layouts (include/fmha_mxfp8.h):
//   fmha_fwd_hd128_mxfp8_v3_vs128             256 query rows / 8 waves per block, whole KV range
//   fmha_fwd_hd128_mxfp8_v3_t128              128 query rows / 4 waves per block
//   fmha_fwd_hd128_mxfp8_v3_kvsplit           256 rows per block over one KV split -> fp16 partials + base-2 LSE
//   fmha_fwd_hd128_mxfp8_v3_kvsplit_combine8h LSE-weighted merge of the partials, 8 outputs per thread
//
// Per wave: 32 query rows. S^T (keys x queries) = K Q^T on v_mfma_scale_f32_32x32x64_f8f6f4 with the E8M0
// scales in the MFMA (K scale byte-selected per lane half, Q scale - 9 so S comes out x 2^-9), seeded with the
// per-query softmax reference b; O^T (dims x queries) += V^T P^T on the same MFMA with unit scales, V^T read
// with ds_read_b64_tr_b8 from a [key][dim] LDS tile; the row sums of the quantised P by a dense 16x16x128 MFMA
// with a constant ones pattern. The C layout of S^T is the B-operand layout of P^T, so P never moves.
//
// Softmax recipe (the reference's, crates/amdgpu-tile/src/softmax.rs:31-323, reduce.rs:66-113):
//   S' = S / 512 + b, b = 4 (hi + lo) kept as two f16 words; per 128-key tile m = rowmax(S');
//   sequences of >= 4 tiles: lazy rebase when !(thr >= m), thr = 0.26135647, target 0.24799132, P scale 1/4;
//   shorter: eager rebase when thr < m, thr = 120/512, target 131/512, LUT-corrected pknorm, P scale 1;
//   P = e4m3(bf16_bits(pknorm_u16(S')) / scale) (a Schraudolph exp2: the u16 read as bf16 is 2^(512 S' - 127)).
//
// K/V/K-scale tiles are staged global -> LDS by global_load_lds_dwordx4 (no VGPR round trip) into a
// double-buffered ring; 16-byte chunk c of LDS row r holds logical chunk c ^ swz(r), which makes both the
// ds_read_b128 K reads and the transposing V reads bank-conflict free.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/fmha_mxfp8.h"

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef short v2s __attribute__((ext_vector_type(2)));
typedef unsigned short v2u16 __attribute__((ext_vector_type(2)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

#define LDS_AS __attribute__((address_space(3)))

namespace {

constexpr int kD = 128;
constexpr int kTile = 128;                    // keys per KV tile
constexpr int kTileBytes = kTile * kD;        // 16 KiB
constexpr int kLdsK = 0;                      // 2 slots
constexpr int kLdsV = 2 * kTileBytes;         // 2 slots
constexpr int kLdsKs = 4 * kTileBytes;        // 2 slots x 512 B
constexpr int kLdsBytes = 4 * kTileBytes + 2 * 512;

struct Prm {
    const uint8_t* q;
    const uint8_t* k;
    const uint8_t* v;
    const uint8_t* qs;
    const uint8_t* ks;
    const float* vd;
    uint8_t* o;
    float* lse_out;
    uint32_t S, SK, H, gqa, flags;
    uint32_t q_seq, q_b, k_seq, k_b, v_seq, v_b, o_seq, o_b, qs_b, ks_b;
    uint8_t* ohat;
    float* lse;
    uint32_t splits, rows_total;
};

__device__ inline Prm prm_from(const fmha_mxfp8_args& a) {
    Prm p;
    p.q = (const uint8_t*)a.ptr_q; p.k = (const uint8_t*)a.ptr_k; p.v = (const uint8_t*)a.ptr_v;
    p.qs = (const uint8_t*)a.ptr_q_descale; p.ks = (const uint8_t*)a.ptr_k_descale; p.vd = (const float*)a.ptr_v_descale;
    p.o = (uint8_t*)a.ptr_o; p.lse_out = (float*)a.ptr_lse;
    p.S = a.s_seq_len; p.SK = a.s_kv_seq_len; p.H = a.s_q_head_num; p.gqa = a.s_gqa; p.flags = a.flags;
    p.q_seq = a.s_Seqs; p.q_b = a.s_Bs; p.k_seq = a.s_k_Seqs; p.k_b = a.s_k_Bs; p.v_seq = a.s_v_Seqs; p.v_b = a.s_v_Bs;
    p.o_seq = a.s_o_Seqs; p.o_b = a.s_o_Bs; p.qs_b = a.s_descale_q_Bs; p.ks_b = a.s_descale_k_Bs;
    p.ohat = nullptr; p.lse = nullptr; p.splits = 1; p.rows_total = 0;
    return p;
}

// LDS chunk swizzle: injective on any 8 consecutive rows and on {r..r+3, r+8..r+11} (r % 4 == 0).
__device__ inline uint32_t swz(uint32_t r) { return (r & 3u) | ((((r >> 2) ^ (r >> 3)) & 1u) << 2); }

__device__ inline uint32_t wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

__device__ inline float h2f(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (unsigned short)(h & 0xffffu)); }
__device__ inline uint32_t f2h(float f) { return (uint32_t)__builtin_bit_cast(unsigned short, (_Float16)f); }

__device__ inline float bias_of(uint32_t w) { return (h2f(w) + h2f(w >> 16)) * 4.0f; }

__device__ inline void dma16(const void* src, uint32_t lds_off) {
    __builtin_amdgcn_global_load_lds(src, (LDS_AS void*)(uintptr_t)lds_off, 16, 0, 0);
}
__device__ inline void dma4(const void* src, uint32_t lds_off) {
    __builtin_amdgcn_global_load_lds(src, (LDS_AS void*)(uintptr_t)lds_off, 4, 0, 0);
}

__device__ inline v4i lds_read16(uint32_t off) { return *(const LDS_AS v4i*)(uintptr_t)off; }
__device__ inline uint32_t lds_read4(uint32_t off) { return *(const LDS_AS uint32_t*)(uintptr_t)off; }

__device__ inline v8i cat8(v4i a, v4i b) { return (v8i){a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]}; }

template <int NT>
struct Stager {
    // global -> LDS staging of one 128-key tile: K and V (16 KiB each, 16 B per lane-instruction) and the
    // K scales (512 B: every wave loads 64 keys' dwords, waves w and w+2 the same ones, so the vmcnt
    // accounting is identical in every wave).
    static constexpr int kN = kTileBytes / (NT * 16);   // instructions per thread per 16 KiB tile
    const uint8_t* kb;   // K of this (batch, kv head)
    const uint8_t* vb;
    const uint8_t* ksb;
    uint32_t k_seq, ks_row, kv_last;
    uint32_t wave, lane;
    uint32_t lds;   // LDS base of the ring

    __device__ void stage(uint32_t key0, uint32_t slot) const {
        {
            const uint32_t key = min(key0 + (wave & 1u) * 64u + lane, kv_last);
            dma4(ksb + (size_t)key * ks_row, lds + kLdsKs + slot * 512u + (wave & 1u) * 256u);
        }
#pragma unroll
        for (int i = 0; i < kN; ++i) {
            const uint32_t base = (uint32_t)(i * NT) * 16u + wave * 1024u;   // wave-uniform LDS offset
            const uint32_t p = base + lane * 16u;
            const uint32_t row = p >> 7, pch = (p >> 4) & 7u;
            const uint32_t key = min(key0 + row, kv_last);
            const size_t g = (size_t)key * k_seq + ((pch ^ swz(row)) << 4);
            dma16(kb + g, lds + kLdsK + slot * kTileBytes + base);
            dma16(vb + g, lds + kLdsV + slot * kTileBytes + base);
        }
    }
    static constexpr int kLoadsPerStage = 2 * kN + 1;
};

// Workgroup barrier that is also a compiler memory barrier (no LDS access moves across it) but, unlike
// __syncthreads, does not drain vmcnt: the next tile's LDS DMA stays in flight across it.
__device__ inline void block_barrier() { asm volatile("s_barrier" ::: "memory"); }

template <int N>
__device__ inline void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Softmax recipe constants (softmax.rs:24-27 exact copy; softmax.rs:80-88 lazy copy).
struct Recipe {
    float thr, b131, conv;
};

// V^T fragment of one PV MFMA: four transposing reads 16 keys apart (2048 B). Issued as one asm block that
// drains lgkmcnt: the compiler's ds_read_tr intrinsic is made to wait for every outstanding LDS DMA (vmcnt(0)),
// which would serialise the next tile's staging with this tile's compute.
__device__ inline v8i lds_read_vt(uint32_t addr) {
    v2i r0, r1, r2, r3;
    asm volatile(
        "ds_read_b64_tr_b8 %0, %4\n\t"
        "ds_read_b64_tr_b8 %1, %4 offset:2048\n\t"
        "ds_read_b64_tr_b8 %2, %4 offset:4096\n\t"
        "ds_read_b64_tr_b8 %3, %4 offset:6144\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(r0), "=&v"(r1), "=&v"(r2), "=&v"(r3)
        : "v"(addr));
    return (v8i){r0[0], r0[1], r1[0], r1[1], r2[0], r2[1], r3[0], r3[1]};
}

// One tile's softmax on the S^T accumulators of a wave: row max (+ partner lane), the rebase decision and
// rescale, and the fp8 P words.
template <bool LUT>
__device__ __forceinline__ void softmax_tile(const Recipe& rc, v16f (&s)[4], v16f (&o)[4], v4f& lacc, v16f& bias, uint32_t& bw,
                                             uint32_t (&pw)[4][4]) {
    float m = -1.0e30f;
#pragma unroll
    for (int t4 = 0; t4 < 4; ++t4)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            m = fmaxf(m, s[t4][i]);
        }
    {
        const auto sw = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, m), __builtin_bit_cast(uint32_t, m), false, false);
        m = fmaxf(__builtin_bit_cast(float, (uint32_t)sw[0]), __builtin_bit_cast(float, (uint32_t)sw[1]));
    }
    // rebase decision (softmax.rs:125-160 eager: thr < m; softmax.rs:186-241 lazy: !(thr >= m), which also takes NaN)
    const bool grow = LUT ? (rc.thr < m) : !(rc.thr >= m);
    if (__builtin_amdgcn_ballot_w64(grow)) {
        const float hi_o = h2f(bw), lo_o = h2f(bw >> 16);
        const float b_old = (hi_o + lo_o) * 4.0f;
        const float tt = rc.b131 - m;
        const float b_new = b_old + tt;
        const float qq = b_new * 0.25f;
        const uint32_t h_raw = f2h(qq);
        const float hq = h2f(h_raw);
        const float r = qq - hq;
        const uint32_t l_raw = f2h(r);
        const float lq = h2f(l_raw);
        const float b_q = (hq + lq) * 4.0f;
        const float delta = grow ? b_q - b_old : 0.0f;
        bw = grow ? (h_raw | (l_raw << 16)) : bw;
#pragma unroll
        for (int t4 = 0; t4 < 4; ++t4)
#pragma unroll
            for (int i = 0; i < 16; ++i) s[t4][i] += delta;
        const float corr = __builtin_amdgcn_exp2f(delta * 512.0f);
#pragma unroll
        for (int dc = 0; dc < 4; ++dc)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[dc][i] *= corr;
#pragma unroll
        for (int i = 0; i < 4; ++i) lacc[i] *= corr;
        const float bnew = bias_of(bw);
#pragma unroll
        for (int i = 0; i < 16; ++i) bias[i] = bnew;
    }
    // P = e4m3(pknorm(S') [- LUT] / scale), 4 keys per word
#pragma unroll
    for (int t4 = 0; t4 < 4; ++t4)
#pragma unroll
        for (int a = 0; a < 4; ++a) {
            float x[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) x[c] = s[t4][4 * a + c];
            v2u16 u01 = __builtin_bit_cast(v2u16, __builtin_amdgcn_cvt_pknorm_u16(x[0], x[1]));
            v2u16 u23 = __builtin_bit_cast(v2u16, __builtin_amdgcn_cvt_pknorm_u16(x[2], x[3]));
            if (LUT) {
                // u -= LUT[(u >> 4) & 7], LUT = {0, 6, 9, 11, 11, 10, 7, 3} (reduce.rs:84-91)
                const uint32_t i01 = (__builtin_bit_cast(uint32_t, u01) >> 4) & 0x00070007u;
                const uint32_t i23 = (__builtin_bit_cast(uint32_t, u23) >> 4) & 0x00070007u;
                u01 = u01 - __builtin_bit_cast(v2u16, __builtin_amdgcn_perm(0x03070a0bu, 0x0b090600u, i01));
                u23 = u23 - __builtin_bit_cast(v2u16, __builtin_amdgcn_perm(0x03070a0bu, 0x0b090600u, i23));
            }
            v2s w = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16((v2s){0, 0}, __builtin_bit_cast(v2bf, u01), rc.conv, false);
            w = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(w, __builtin_bit_cast(v2bf, u23), rc.conv, true);
            pw[t4][a] = __builtin_bit_cast(uint32_t, w);
        }
}

// The per-wave attention state over one key range [key_lo, key_hi) of one block.
template <int NT, bool LUT, bool SPLIT>
__device__ void attend(const Prm& p, uint32_t lds, uint32_t qtile, uint32_t head, uint32_t bidx, uint32_t split, uint32_t key_lo,
                       uint32_t key_hi) {
    constexpr int ROWS = NT / 64 * 32;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = wave_id();
    const uint32_t n = lane & 31u, hh = lane >> 5;
    const Recipe rc = LUT ? Recipe{120.0f / 512.0f, 131.0f / 512.0f, 1.0f}
                          : Recipe{__builtin_bit_cast(float, 0x3e85d086u), __builtin_bit_cast(float, 0x3e7df17eu), 0.25f};
    const uint32_t kvh = head / p.gqa;
    const uint32_t row0 = qtile * ROWS + wave * 32u;
    const uint32_t row = row0 + n;
    const uint32_t row_c = min(row, p.S - 1u);
    const bool causal = (p.flags & 1u) != 0;

    // ---- Q fragments (B operand of the QK MFMA, resident) and their scales
    const uint8_t* qrow = p.q + (size_t)bidx * p.q_b + (size_t)row_c * p.q_seq + head * kD;
    v8i qf[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const v4i a = *(const v4i*)(qrow + 64 * c + 16 * hh);
        const v4i b = *(const v4i*)(qrow + 64 * c + 32 + 16 * hh);
        qf[c] = cat8(a, b);
    }
    const uint32_t qsw = *(const uint32_t*)(p.qs + (size_t)bidx * p.qs_b + (size_t)row_c * (p.H * 4u) + head * 4u);
    int sq[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) sq[c] = (int)(((qsw >> (8 * (2 * c + hh))) - 9u) & 0xffu);
    const float vd = *p.vd;

    // ---- causal limits: query row i sees keys [0, i + SK - S + 1)
    uint32_t lim_row = key_hi, lim_wave_min = key_hi, lim_wave_max = key_hi, lim_blk_max = key_hi;
    if (causal) {
        const int off = (int)p.SK - (int)p.S + 1;
        lim_row = (uint32_t)max(0, min((int)key_hi, (int)row + off));
        lim_wave_min = (uint32_t)max(0, min((int)key_hi, (int)row0 + off));
        lim_wave_max = (uint32_t)max(0, min((int)key_hi, (int)row0 + 31 + off));
        lim_blk_max = (uint32_t)max(0, min((int)key_hi, (int)(qtile * ROWS + ROWS - 1) + off));
    }
    const uint32_t key_end = causal ? min(key_hi, lim_blk_max) : key_hi;   // block's last useful key + 1
    const uint32_t ntiles = key_end > key_lo ? (key_end - key_lo + kTile - 1) / kTile : 0;

    Stager<NT> st;
    st.kb = p.k + (size_t)bidx * p.k_b + kvh * kD;
    st.vb = p.v + (size_t)bidx * p.v_b + kvh * kD;
    st.k_seq = p.k_seq;
    st.ks_row = p.k_seq >> 5;
    st.ksb = p.ks + (size_t)bidx * p.ks_b + kvh * 4u;
    st.kv_last = p.SK - 1u;
    st.wave = wave;
    st.lane = lane;
    st.lds = lds;

    // ---- per-lane LDS addresses
    // K fragment (A operand, lane = key row n of the 32-key block, half hh): chunks 4c + 2e + hh of row n
    uint32_t kaddr[2][2];
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int e = 0; e < 2; ++e) kaddr[c][e] = n * 128u + (((uint32_t)(4 * c + 2 * e) + hh) ^ swz(n)) * 16u;
    // V^T fragment via ds_read_b64_tr_b8: source lane (g, jj, pp) reads key 16 r + rlo of the 64-key half,
    // dims 32 dc + 16 (g & 1) + 8 pp .. +7
    uint32_t vaddr[4];
    {
        const uint32_t g = lane >> 4, jj = (lane >> 1) & 7u, pp = lane & 1u;
        const uint32_t rlo = 8u * (jj >> 2) + 4u * (g >> 1) + (jj & 3u);
#pragma unroll
        for (int dc = 0; dc < 4; ++dc) vaddr[dc] = rlo * 128u + ((((uint32_t)(2 * dc)) + (g & 1u)) ^ swz(rlo)) * 16u + 8u * pp;
    }
    // ones pattern of the row-sum MFMA (16x16x128): lane la holds A row la % 16, k-groups la / 16; row m sums
    // the P bytes of query (m % 2 ? n + 16 : n) -> ones iff (la / 16) % 2 == la % 2
    const int onew = (((lane >> 4) & 1u) == (lane & 1u)) ? 0x38383838 : 0;
    const v8i ones = (v8i){onew, onew, onew, onew, onew, onew, onew, onew};

    // ---- state
    uint32_t bw = 0x48004800u;   // two f16 words (hi = low half); b = 64 makes tile 0 rebase
    v16f bias;
    {
        const float b0 = bias_of(bw);
#pragma unroll
        for (int i = 0; i < 16; ++i) bias[i] = b0;
    }
    v16f o[4];
#pragma unroll
    for (int dc = 0; dc < 4; ++dc)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[dc][i] = 0.0f;
    v4f lacc = {0.0f, 0.0f, 0.0f, 0.0f};

    if (ntiles > 0) st.stage(key_lo, 0);
    for (uint32_t it = 0; it < ntiles; ++it) {
        const uint32_t slot = it & 1u;
        const uint32_t key0 = key_lo + it * kTile;
        if (it + 1 < ntiles) {
            st.stage(key0 + kTile, slot ^ 1u);
            wait_vmcnt<Stager<NT>::kLoadsPerStage>();
        } else {
            wait_vmcnt<0>();
        }
        block_barrier();

        const uint32_t kbase = lds + kLdsK + slot * kTileBytes;
        const uint32_t vbase = lds + kLdsV + slot * kTileBytes;
        const uint32_t ksbase = lds + kLdsKs + slot * 512u;
        // keys of this tile valid for this lane: < kv end of the range, < causal limit
        const uint32_t vlim = min(key_hi, lim_row);
        const bool wave_skip = causal && key0 >= lim_wave_max;   // every key of the tile is past the wave's last visible key
        if (!wave_skip) {
            // ---- S^T = K Q^T (scaled MFMA, 2 per 32-key block), seeded with the reference b
            v16f s[4];
#pragma unroll
            for (int t4 = 0; t4 < 4; ++t4) {
                const uint32_t ksw = lds_read4(ksbase + (32u * t4 + n) * 4u) >> (8u * hh);
                const v8i kf0 = cat8(lds_read16(kbase + 4096u * t4 + kaddr[0][0]), lds_read16(kbase + 4096u * t4 + kaddr[0][1]));
                const v8i kf1 = cat8(lds_read16(kbase + 4096u * t4 + kaddr[1][0]), lds_read16(kbase + 4096u * t4 + kaddr[1][1]));
                // d 0..63 then d 64..127; op_sel picks K-scale byte 2c of the lane-half-shifted word
                s[t4] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(kf0, qf[0], bias, 0, 0, 0, (int)ksw, 0, sq[0]);
                s[t4] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(kf1, qf[1], s[t4], 0, 0, 2, (int)ksw, 0, sq[1]);
            }
            // ---- softmax: row max, rebase, P (the masked form only on tiles that cross the range end / causal limit)
            uint32_t pw[4][4];
            if (key0 + kTile > min(key_hi, lim_wave_min)) {
                // keys at or past the range end / causal limit: -1e30 takes no part in the max and converts to P = 0
                // (pknorm clamps), the reference's two fills (reduce.rs:13-49) in one
                const int nvalid = (int)vlim - (int)key0 - 4 * (int)hh;
#pragma unroll
                for (int t4 = 0; t4 < 4; ++t4)
#pragma unroll
                    for (int i = 0; i < 16; ++i)
                        s[t4][i] = (32 * t4 + 8 * (i >> 2) + (i & 3)) < nvalid ? s[t4][i] : -1.0e30f;
            }
            softmax_tile<LUT>(rc, s, o, lacc, bias, bw, pw);
            // ---- row sums of P and O^T += V^T P^T, one 64-key half at a time
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const v8i pf = (v8i){(int)pw[2 * j][0], (int)pw[2 * j][1], (int)pw[2 * j][2], (int)pw[2 * j][3],
                                     (int)pw[2 * j + 1][0], (int)pw[2 * j + 1][1], (int)pw[2 * j + 1][2], (int)pw[2 * j + 1][3]};
                lacc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(ones, pf, lacc, 0, 0, 0, 127, 0, 127);
#pragma unroll
                for (int dc = 0; dc < 4; ++dc) {
                    const v8i vf = lds_read_vt(vbase + vaddr[dc] + 8192u * j);
                    o[dc] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(vf, pf, o[dc], 0, 0, 0, 127, 0, 127);
                }
            }
        }
        block_barrier();
    }

    // ---- epilogue
    const float l = ((lane >> 4) & 1u) ? lacc[1] : lacc[0];   // the lane's query row sum (see the ones pattern)
    if (!SPLIT) {
        const float fin = __builtin_amdgcn_rcpf(l) * vd;   // state.rs:79-83
        if (row < p.S) {
            uint8_t* orow = p.o + (size_t)bidx * p.o_b + (size_t)row * p.o_seq + head * 256u;
#pragma unroll
            for (int dc = 0; dc < 4; ++dc)
#pragma unroll
                for (int a = 0; a < 4; ++a) {
                    const v2bf w0 = {(__bf16)(o[dc][4 * a] * fin), (__bf16)(o[dc][4 * a + 1] * fin)};
                    const v2bf w1 = {(__bf16)(o[dc][4 * a + 2] * fin), (__bf16)(o[dc][4 * a + 3] * fin)};
                    const v2i pk = {__builtin_bit_cast(int, w0), __builtin_bit_cast(int, w1)};
                    *(v2i*)(orow + (32 * dc + 8 * a + 4 * hh) * 2) = pk;
                }
            if (p.lse_out && hh == 0) {
                // natural-log LSE of the scores (extension): P = 2^(S + 512 b - 127) / conv, l = sum P
                const float hl = h2f(bw) + h2f(bw >> 16);
                const float lse2 = __builtin_amdgcn_logf(l) - hl * 2048.0f + 127.0f + __builtin_amdgcn_logf(rc.conv);
                p.lse_out[((size_t)bidx * p.H + head) * p.S + row] = lse2 * 0.69314718055994531f;
            }
        }
    } else {
        // block3.rs:291-356 / softmax.rs:308-322: Ohat = (O / 16) * (v_descale / l_total), l_total = l / 16;
        // lse = log2(l_total) - 2048 (hi + lo)
        const float l_total = l * 0.0625f;
        const float fin = __builtin_amdgcn_rcpf(l_total) * vd;
        if (row < p.S) {
            const size_t prow = (size_t)split * p.rows_total + ((size_t)bidx * p.S + row) * p.H + head;
            uint8_t* orow = p.ohat + prow * 256u;
#pragma unroll
            for (int dc = 0; dc < 4; ++dc)
#pragma unroll
                for (int a = 0; a < 4; ++a) {
                    uint32_t w[2];
#pragma unroll
                    for (int c = 0; c < 2; ++c) {
                        const uint32_t lo16 = f2h((o[dc][4 * a + 2 * c] * 0.0625f) * fin);
                        const uint32_t hi16 = f2h((o[dc][4 * a + 2 * c + 1] * 0.0625f) * fin);
                        w[c] = lo16 | (hi16 << 16);
                    }
                    *(v2i*)(orow + (32 * dc + 8 * a + 4 * hh) * 2) = (v2i){(int)w[0], (int)w[1]};
                }
            if (hh == 0) {
                const float hl = h2f(bw) + h2f(bw >> 16);
                p.lse[prow] = __builtin_amdgcn_logf(l_total) + (hl * 2048.0f) * -1.0f;
            }
        }
    }
}

// Workgroup -> (q tile, head, z): consecutive tiles of one (batch, head) land on one XCD (the hardware deals
// workgroups round-robin over the 8 XCDs), so each XCD's L2 holds the K/V its blocks share.
__device__ inline void block_coords(uint32_t& qt, uint32_t& head, uint32_t& z) {
    // grid extents from the AQL dispatch packet (grid_size in work-items at byte 12/16/20, workgroup_size at 4/6/8),
    // so the kernels need no hidden kernel arguments: the kernarg segment is exactly the reference's
    const uint8_t __attribute__((address_space(4)))* pk = (const uint8_t __attribute__((address_space(4)))*)__builtin_amdgcn_dispatch_ptr();
    const uint32_t wgx = *(const uint16_t __attribute__((address_space(4)))*)(pk + 4);
    const uint32_t gx = *(const uint32_t __attribute__((address_space(4)))*)(pk + 12) / wgx;
    const uint32_t gy = *(const uint32_t __attribute__((address_space(4)))*)(pk + 16);
    const uint32_t gz = *(const uint32_t __attribute__((address_space(4)))*)(pk + 20);
    const uint32_t nblk = gx * gy * gz;
    uint32_t L = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
    if ((nblk & 7u) == 0u) L = (L & 7u) * (nblk >> 3) + (L >> 3);
    qt = L % gx;
    const uint32_t rest = L / gx;
    head = rest % gy;
    z = rest / gy;
}

template <int NT>
__device__ void full_kernel(const fmha_mxfp8_args& a, uint32_t lds) {
    const Prm p = prm_from(a);
    uint32_t qt, head, z;
    block_coords(qt, head, z);
    const bool lut = (p.SK + 127u) / 128u < 4u;   // state.rs:75-77
    if (lut) attend<NT, true, false>(p, lds, qt, head, z, 0, 0, p.SK);
    else attend<NT, false, false>(p, lds, qt, head, z, 0, 0, p.SK);
}

}  // namespace

#define FMHA_LDS_BASE(name)                                                 \
    __shared__ __attribute__((aligned(1024))) uint8_t name[kLdsBytes]; \
    const uint32_t name##_base = (uint32_t)(uintptr_t)(LDS_AS uint8_t*)name

extern "C" __global__ void __launch_bounds__(512, 1) fmha_fwd_hd128_mxfp8_v3_vs128(fmha_mxfp8_args a) {
    FMHA_LDS_BASE(smem);
    full_kernel<512>(a, smem_base);
}

extern "C" __global__ void __launch_bounds__(256, 1) fmha_fwd_hd128_mxfp8_v3_t128(fmha_mxfp8_args a) {
    FMHA_LDS_BASE(smem);
    full_kernel<256>(a, smem_base);
}

extern "C" __global__ void __launch_bounds__(512, 1) fmha_fwd_hd128_mxfp8_v3_kvsplit(fmha_mxfp8_kvsplit_args ka) {
    FMHA_LDS_BASE(smem);
    const fmha_mxfp8_args& a = *reinterpret_cast<const fmha_mxfp8_args*>(&ka);   // bytes 0x000..0x26F are the base layout
    Prm p = prm_from(a);
    p.flags = 0;   // 0x280 holds the split count in this layout
    p.lse_out = nullptr;
    p.ohat = (uint8_t*)ka.ptr_ohat;
    p.lse = (float*)ka.ptr_lse;
    p.splits = ka.kvs_splits;
    p.rows_total = ka.kvs_rows_total;
    uint32_t qt, head, z;
    block_coords(qt, head, z);
    // components.rs:20-30 / 58-74: z = batch * splits + split; split s owns tiles [s tps, min(ntiles, (s+1) tps))
    const uint32_t bidx = z / p.splits, split = z % p.splits;
    const uint32_t ntiles = (p.SK + 127u) / 128u;
    const uint32_t tps = (ntiles + p.splits - 1u) / p.splits;
    const uint32_t tile_lo = split * tps;
    const uint32_t tile_hi = min(ntiles, tile_lo + tps);
    const uint32_t key_lo = tile_lo * 128u, key_hi = min(tile_hi * 128u, p.SK);
    const bool lut = ntiles < 4u;
    if (lut) attend<512, true, true>(p, smem_base, qt, head, bidx, split, key_lo, key_hi);
    else attend<512, false, true>(p, smem_base, qt, head, bidx, split, key_lo, key_hi);
}

// epilogue.rs:89-167 / io.rs:164-185: thread t -> 8 consecutive outputs of row t >> 4 (tail threads redo the last group)
extern "C" __global__ void __launch_bounds__(256) fmha_fwd_hd128_mxfp8_v3_kvsplit_combine8h(fmha_mxfp8_combine_args a) {
    const uint32_t rows = a.rows_total, splits = a.splits;
    const uint32_t groups = rows << 4;
    uint32_t t = blockIdx.x * 256u + threadIdx.x;
    t = t < groups ? t : groups - 1u;
    const uint32_t row = t >> 4;
    const float* lse = (const float*)a.ptr_lse;
    const uint8_t* ohat = (const uint8_t*)a.ptr_ohat;
    float m = -1.0e30f, den = 0.0f;
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
    for (uint32_t s = 0; s < splits; ++s) {
        const size_t rs = (size_t)s * rows;
        const float l = lse[rs + row];
        const v4i ov = *(const v4i*)(ohat + ((rs << 4) + t) * 16u);
        const float m_new = fmaxf(m, l);
        const float dm = m_new * -1.0f;
        const float al = __builtin_amdgcn_exp2f(m + dm);
        const float w = __builtin_amdgcn_exp2f(l + dm);
        den = den * al + w;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            acc[2 * i] = acc[2 * i] * al + w * h2f((uint32_t)ov[i]);
            acc[2 * i + 1] = acc[2 * i + 1] * al + w * h2f((uint32_t)ov[i] >> 16);
        }
        m = m_new;
    }
    const float rd = __builtin_amdgcn_rcpf(den);
    v4i outv;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const v2bf w = {(__bf16)(acc[2 * i] * rd), (__bf16)(acc[2 * i + 1] * rd)};
        outv[i] = __builtin_bit_cast(int, w);
    }
    *(v4i*)((uint8_t*)a.ptr_out + (size_t)t * 16u) = outv;
}
