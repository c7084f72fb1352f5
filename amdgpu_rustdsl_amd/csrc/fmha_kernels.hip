// fmha_kernels.hip - MXFP8 FMHA forward, head dim 128, hand-written HIP for gfx950 (MI355X).
//
// Four kernels with the reference's names and kernarg layouts (include/fmha_mxfp8.h):
//   fmha_fwd_hd128_mxfp8_v3_vs128             256 query rows / 8 waves per block, whole KV range
//   fmha_fwd_hd128_mxfp8_v3_t128              128 query rows / 4 waves per block
//   fmha_fwd_hd128_mxfp8_v3_kvsplit           256 rows per block over one KV split -> fp16 partials + base-2 LSE
//   fmha_fwd_hd128_mxfp8_v3_kvsplit_combine8h LSE-weighted merge of the partials, 8 outputs per thread
// and extensions with the same layouts: _t128_split_tiles (t128's grid, 8 waves splitting each tile's keys),
// _kvsplit_combine_wide (the merge for many partials), and the _scaled kernels (the softmax scale applied in the kernel).
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
// K/V tiles reach a 4-slot LDS ring (the 256-thread t128 uses 3 of the slots) by direct HBM -> LDS copies
// (buffer_load_dwordx4 ... lds); 16-byte chunk c of LDS row r holds logical chunk c ^ swz(r), which makes both the
// ds_read_b128 K reads and the transposing V reads bank-conflict free. The 512-thread kernels stage the K-scale words
// through registers (the upper k-group reads a copy shifted by one byte), the 256-thread kernel copies them directly.
// The Q fragments stay in registers.

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <type_traits>
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
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef float v2f __attribute__((ext_vector_type(2)));

#define LDS_AS __attribute__((address_space(3)))
// wave issue priority around the MFMA phases
#define FMHA_SETPRIO(x) __builtin_amdgcn_s_setprio(x)
#define GLOBAL_AS __attribute__((address_space(1)))

namespace {

#ifndef FMHA_PREFETCH
#define FMHA_PREFETCH 2
#endif

constexpr int kD = 128;
constexpr int kTile = 128;                    // keys per KV tile
constexpr int kTileBytes = kTile * kD;        // 16 KiB
constexpr int kSlots = 4;                     // ring depth of the direct-copy path (t128 uses 3 of the slots)
constexpr int kLdsK = 0;                      // kSlots K tiles
constexpr int kLdsV = kSlots * kTileBytes;    // kSlots V tiles
constexpr int kLdsKs = 2 * kSlots * kTileBytes;   // kSlots x 1 KiB of K scales: the words, then the words >> 8
constexpr int kKsSlot = 1024;
constexpr int kLdsKsDummy = kLdsKs + kSlots * kKsSlot;   // 1 KiB sink for the K-scale writes of threads 256..511
// per-32-key V scales (extension): kSlots x 512 B (4 blocks of 32 keys x 128 columns), then a 2 KiB sink for the
// copies of the waves that carry none
constexpr int kVsSlot = 512;
constexpr int kLdsVs = kLdsKsDummy + 1024;
constexpr int kLdsVsSink = kLdsVs + kSlots * kVsSlot;
// epilogue staging of the output rows (after the loop, over the dead ring): 32 rows of 272 B per wave, above the
// 68 KiB the split-tile merge uses
constexpr int kLdsEpi = 68 * 1024;
constexpr int kEpiRow = 272;
// the ping-pong kernels' group B stages its rows apart from the ring while group A still reads it: 16 rows of 272 B
// per wave slot at a time, 4 slots
constexpr int kLdsTail = kLdsVsSink + 2048;
constexpr int kLdsBytes = kLdsTail + 4 * 16 * kEpiRow;
static_assert(kLdsEpi + 8 * 32 * kEpiRow <= kLdsTail, "epilogue staging fits");
static_assert(kLdsBytes <= 160 * 1024, "LDS of one workgroup");

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
    uint32_t f32_partials;   // kvsplit extension: partial rows as f32 (512 B) instead of fp16 (256 B)
    // extension: per-32-key V scales; ptr_v_descale then holds E8M0 [B, ceil(SK/32), HK, 128] (vs_row = HK 128 bytes per
    // 32-key block, vs_b = ceil(SK/32) vs_row per batch) and the per-tensor descale is 1
    const uint8_t* vs32;
    uint32_t vs_row, vs_b;
    // extension: the softmax scale applied in the kernel. c = f32(scale log2 e) = 2^qk_e qk_m, qk_m in [1, 2): qk_e
    // is added to the Q scale exponents, S is seeded with b qk_rm (qk_rm = 1 / qk_m) and multiplied by qk_m. Without
    // the extension qk_e = 0 and qk_m = qk_rm = 1 (the seed is b, exactly).
    float qk_m, qk_rm;
    int32_t qk_e;
    uint32_t qk_scaled;
#ifdef FMHA_TRACE
    uint64_t* trace;   // debug builds only: per (block, wave) timestamps, pointer at kernarg 0x288
    uint64_t t_entry;  // timestamp of the kernel's first instruction
#endif
};

// Debug builds (-DFMHA_TRACE) record s_memrealtime (100 MHz) at phase boundaries: slot i of wave w of logical block
// blk at trace[(blk * 8 + w) * 8 + i], written by lane 0 with a vector store. Release builds compile it away.
#ifdef FMHA_TRACE
#define FMHA_MARK(p, blk, i)                                                                                  \
    do {                                                                                                    \
        if ((p).trace && (threadIdx.x & 63u) == 0u)                                                         \
            (p).trace[((size_t)(blk) * 8u + (threadIdx.x >> 6)) * 8u + (i)] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
// loop marks: the shader-clock cycles between consecutive marks are summed per mark index k (k = 0..3) over tiles
// 4 <= t < ntiles - 2 in scalar registers (no VGPRs in the loop) and written by FMHA_LFLUSH behind the first region
#define FMHA_LMARK(p, blk, t, k)                                                                                  \
    do {                                                                                                        \
        const uint64_t now_ = __builtin_amdgcn_s_memtime();                                                     \
        if ((t) >= 4u && (t) + 2u < ntiles) prof_acc[k] += now_ - prof_last;                                    \
        prof_last = now_;                                                                                       \
    } while (0)
#define FMHA_LFLUSH(p, blk)                                                                                       \
    do {                                                                                                        \
        if ((p).trace && (threadIdx.x & 63u) == 0u)                                                             \
            for (int k_ = 0; k_ < 4; ++k_)                                                                      \
                (p).trace[65536u + ((size_t)(blk) * 8u + (threadIdx.x >> 6)) * 8u + k_] = prof_acc[k_];         \
    } while (0)
#define FMHA_LDECL uint64_t prof_acc[4] = {0, 0, 0, 0}; uint64_t prof_last = 0
#else
#define FMHA_MARK(p, blk, i) do { } while (0)
#define FMHA_LMARK(p, blk, t, k) do { } while (0)
#define FMHA_LFLUSH(p, blk) do { } while (0)
#define FMHA_LDECL do { } while (0)
#endif

#define KA_AS __attribute__((address_space(4)))

// The kernel arguments are read field by field through the kernarg segment pointer, in the constant address space and
// at each field's natural alignment: scalar loads through the scalar cache. (Through the by-value parameter of the
// packed ABI struct the compiler cannot prove alignment and emits vector loads per field and wave, which for 2048 waves
// took microseconds before the first tile.)
template <typename T>
__device__ inline T ka(uint32_t off) {
    return *(const KA_AS T*)((const KA_AS uint8_t*)__builtin_amdgcn_kernarg_segment_ptr() + off);
}
#define KA_FIELD(T, field) ka<T>(offsetof(fmha_mxfp8_args, field))

// The kernel arguments span ten 64-byte lines (0x000-0x28F), and the segment is fresh from the host for every launch,
// so every line misses the caches. Left to itself the compiler reads the fields in three dependent batches (it spills
// some into VGPR lanes between them), each batch touching new lines: three memory round trips before the first tile
// load. One scalar load per line, all in flight together and waited for once, brings every line into the scalar cache
// in a single round trip; the field reads that follow hit it. (Scalar loads only: nothing is written.)
__device__ __forceinline__ void kernarg_lines_touch() {
    uint32_t t0, t1, t2, t3, t4, t5, t6, t7, t8, t9;
    asm volatile(
        "s_load_dword %0, %10, 0x0\n\t"
        "s_load_dword %1, %10, 0x40\n\t"
        "s_load_dword %2, %10, 0x80\n\t"
        "s_load_dword %3, %10, 0xc0\n\t"
        "s_load_dword %4, %10, 0x100\n\t"
        "s_load_dword %5, %10, 0x140\n\t"
        "s_load_dword %6, %10, 0x180\n\t"
        "s_load_dword %7, %10, 0x200\n\t"
        "s_load_dword %8, %10, 0x240\n\t"
        "s_load_dword %9, %10, 0x280\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=s"(t0), "=s"(t1), "=s"(t2), "=s"(t3), "=s"(t4), "=s"(t5), "=s"(t6), "=s"(t7), "=s"(t8), "=s"(t9)
        : "s"(__builtin_amdgcn_kernarg_segment_ptr())
        : "memory");
    (void)t0; (void)t1; (void)t2; (void)t3; (void)t4; (void)t5; (void)t6; (void)t7; (void)t8; (void)t9;
}

// c = f32(softmax scale (kernarg 0x050) x log2 e) split into 2^e m (the host checked that it is a positive normal)
__device__ inline void set_qk_scale(Prm& p, bool on) {
    p.qk_scaled = on ? 1u : 0u;
    p.qk_e = 0;
    p.qk_m = p.qk_rm = 1.0f;
    if (!on) return;
    const float c = ka<float>(0x050) * 1.44269504088896340736f;
    const uint32_t u = __builtin_bit_cast(uint32_t, c);
    p.qk_e = (int32_t)((u >> 23) & 0xffu) - 127;
    p.qk_m = __builtin_bit_cast(float, (u & 0x007fffffu) | (127u << 23));
    p.qk_rm = 1.0f / p.qk_m;
}

// SC: the `_scaled` kernels, which apply the softmax scale at 0x050; the reference-named kernels fold qk_m = qk_rm = 1,
// qk_e = 0 as constants (their code carries nothing of the extension).
template <bool SC = false, bool KVS = false>
__device__ inline Prm prm_from_kernarg() {
    kernarg_lines_touch();
    Prm p;
    p.q = (const uint8_t*)KA_FIELD(uint64_t, ptr_q); p.k = (const uint8_t*)KA_FIELD(uint64_t, ptr_k);
    p.v = (const uint8_t*)KA_FIELD(uint64_t, ptr_v);
    p.qs = (const uint8_t*)KA_FIELD(uint64_t, ptr_q_descale); p.ks = (const uint8_t*)KA_FIELD(uint64_t, ptr_k_descale);
    p.vd = (const float*)KA_FIELD(uint64_t, ptr_v_descale);
    p.o = (uint8_t*)KA_FIELD(uint64_t, ptr_o); p.lse_out = (float*)KA_FIELD(uint64_t, ptr_lse);
    p.S = KA_FIELD(uint32_t, s_seq_len); p.SK = KA_FIELD(uint32_t, s_kv_seq_len); p.H = KA_FIELD(uint32_t, s_q_head_num);
    p.gqa = KA_FIELD(uint32_t, s_gqa); p.flags = KA_FIELD(uint32_t, flags);
    p.q_seq = KA_FIELD(uint32_t, s_Seqs); p.q_b = KA_FIELD(uint32_t, s_Bs); p.k_seq = KA_FIELD(uint32_t, s_k_Seqs);
    p.k_b = KA_FIELD(uint32_t, s_k_Bs); p.v_seq = KA_FIELD(uint32_t, s_v_Seqs); p.v_b = KA_FIELD(uint32_t, s_v_Bs);
    p.o_seq = KA_FIELD(uint32_t, s_o_Seqs); p.o_b = KA_FIELD(uint32_t, s_o_Bs);
    p.qs_b = KA_FIELD(uint32_t, s_descale_q_Bs); p.ks_b = KA_FIELD(uint32_t, s_descale_k_Bs);
    p.vs32 = (p.flags & FMHA_FLAG_V_SEQ32) ? (const uint8_t*)p.vd : nullptr;
    p.vs_row = p.k_seq;
    p.vs_b = ((p.SK + 31u) >> 5) * p.vs_row;
    p.ohat = nullptr; p.lse = nullptr; p.splits = 1; p.rows_total = 0; p.f32_partials = 0;
    set_qk_scale(p, SC);
#ifdef FMHA_TRACE
    // the trace buffer: 0x288 of the 656-byte layout; the KV split's 648-byte layout ends there, so it reads the
    // unused 0x040 slot instead
    if (KVS) p.trace = (uint64_t*)(uintptr_t)ka<uint64_t>(0x040);
    else p.trace = (uint64_t*)(uintptr_t)(ka<uint32_t>(0x288) | ((uint64_t)ka<uint32_t>(0x28C) << 32));
#endif
    return p;
}

// LDS chunk swizzle: 16-byte chunk c of tile row r sits at chunk c ^ swz(r), swz(r) = (r2, r1, r3) as bits 0..2.
// Bank-conflict free (measured with SQ_LDS_BANK_CONFLICT on gfx950) for both readers: the K ds_read_b128 (lanes =
// 32 consecutive rows, one chunk; needs bits r1, r2, r3 to map to independent chunk bits) and the transposing V
// reads (rows {0-3, 8-11} (+4) with two chunks; needs r1, r3 independent in chunk bits 1-2).
__device__ inline uint32_t swz(uint32_t r) { return ((r >> 2) & 1u) | (r & 2u) | (((r >> 3) & 1u) << 2); }

__device__ inline uint32_t wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

__device__ inline float h2f(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (unsigned short)(h & 0xffffu)); }
__device__ inline uint32_t f2h(float f) { return (uint32_t)__builtin_bit_cast(unsigned short, (_Float16)f); }

__device__ inline float bias_of(uint32_t w) { return (h2f(w) + h2f(w >> 16)) * 4.0f; }

// LDS byte offset of ring slot `slot` of the region at `region`, as an opaque wave-uniform value: loop strength
// reduction cannot see through readfirstlane, so it does not turn every (slot base + per-lane offset) address
// into its own induction variable (one VGPR each, which spilled).
__device__ inline uint32_t slot_base(uint32_t lds, uint32_t region, uint32_t slot, uint32_t slot_bytes) {
    return __builtin_amdgcn_readfirstlane(lds + region + slot * slot_bytes);
}

// uniform base + per-lane offset as one opaque VGPR: constant offsets added to it afterwards fold into the LDS
// instruction's immediate (left to itself the compiler reassociates base + constant first, one add per read).
// The add is the compiler's own and the empty asm only hides its value: a VGPR written by an instruction inside
// inline asm is outside the compiler's hazard checks, and a register whose MFMA result is dead but still in flight
// (the row-sum MFMA's unused dwords) can be handed to it and overwritten by the MFMA's late write.
__device__ inline uint32_t lane_addr(uint32_t uniform_base, uint32_t lane_off) {
    uint32_t r = uniform_base + lane_off;
    asm("" : "+v"(r));
    return r;
}

__device__ inline v4i lds_read16(uint32_t off) { return *(const LDS_AS v4i*)(uintptr_t)off; }
__device__ inline uint32_t lds_read4(uint32_t off) { return *(const LDS_AS uint32_t*)(uintptr_t)off; }

// A 16-byte vector store with system coherence (sc0 sc1: written through the L2), for every row the attention and
// combine kernels write: the output rows and the KV split's partial rows. Written through, they leave no dirty lines
// for the kernel-end write-back of the L2, which otherwise runs after the last wave. Measured on MI355X, identical
// results: cfg2 (B4H8S2048, 16 MiB of output) 33.6 -> 31.4 us, B1H8S8192 -2 %, the 128-row kernels -2 to -4 %, the KV
// split + combine pair 2-4 % on the 256-row shapes, and the combine's own rows -1.3 % more at B1H8S4096 (2 splits).
// The s_nop is the wait state a VALU write of the data registers needs after a VMEM store of more than 8 bytes; the
// compiler adds it after its own stores but not after inline asm.
__device__ inline void store16_system(void* ptr, v4i x) {
    asm volatile("global_store_dwordx4 %0, %1, off sc0 sc1\n\ts_nop 1" ::"v"(ptr), "v"(x) : "memory");
}

// The same for one word (the LSE outputs).
__device__ inline void store4_system(void* ptr, float x) {
    asm volatile("global_store_dword %0, %1, off sc0 sc1" ::"v"(ptr), "v"(x) : "memory");
}

__device__ inline v2i lds_read_tr8(uint32_t off) { return __builtin_amdgcn_ds_read_tr8_b64_v2i32((LDS_AS v2i*)(uintptr_t)off); }

typedef float v8f __attribute__((ext_vector_type(8)));
// Splats in 64-bit halves: one move makes the pair (x, x), then v_mov_b64 copies the pair; each copy goes through an
// empty asm, so that the compiler keeps it a 64-bit copy instead of splitting it into 32-bit moves (the bias seed of S
// and the ones operand: 10 fewer VALU instructions per tile and wave, cfg2 and cfg3 -0.3 %).
typedef unsigned long long v4u64 __attribute__((ext_vector_type(4)));
typedef unsigned long long v8u64 __attribute__((ext_vector_type(8)));
__device__ inline unsigned long long pair2(float x) {
    const unsigned long long u = __builtin_bit_cast(uint32_t, x);
    return u | (u << 32);
}
__device__ inline unsigned long long opq(unsigned long long q) { asm volatile("" : "+v"(q)); return q; }
__device__ inline v8f splat8(float x) {
    const unsigned long long q = pair2(x);
    return __builtin_bit_cast(v8f, (v4u64){q, opq(q), opq(q), opq(q)});
}
__device__ inline v16f splat16(float x) {
    const unsigned long long q = pair2(x);
    return __builtin_bit_cast(v16f, (v8u64){q, opq(q), opq(q), opq(q), opq(q), opq(q), opq(q), opq(q)});
}
__device__ inline v8i cat8(v4i a, v4i b) { return (v8i){a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]}; }

__device__ inline const uint8_t* uniform_ptr(const uint8_t* p) {
    const uint64_t a = (uint64_t)(uintptr_t)p;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)a);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
    return (const uint8_t*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

// Buffer resource over [base, base + bytes): the staging loads are range-checked by the hardware (an
// out-of-range lane reads zeros) on top of the explicit key clamp of the last tile. The base and size are
// wave-uniform by construction; readfirstlane states it so the resource lives in SGPRs (a resource the compiler
// cannot prove uniform costs a waterfall loop per load).
__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    const uint64_t a = (uint64_t)(uintptr_t)base;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a), hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
    void* ub = (void*)(uintptr_t)(((uint64_t)hi << 32) | lo);
    return __builtin_amdgcn_make_buffer_rsrc(ub, (short)0, (int)__builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}

__device__ inline void lds_write16(uint32_t off, v4i v) { *(LDS_AS v4i*)(uintptr_t)off = v; }
__device__ inline void lds_write4(uint32_t off, uint32_t v) { *(LDS_AS uint32_t*)(uintptr_t)off = v; }

// One direct HBM -> LDS copy of 16 bytes per lane: lane L's bytes land at LDS address lds_base + 16 L. Written as inline
// assembly so that the compiler does not see an LDS write: through the builtin it makes every later LDS read of the ring
// wait for all outstanding copies (vmcnt(0)), which would expose their full latency once per phase. The ordering is
// explicit instead: a copy is published by the barrier that follows the wait on its vmcnt (block_barrier_keep_dma).
// M0 carries the LDS base and is declared clobbered. The compiler reserves M0 and keeps no value in it across an asm
// statement of its own accord; build.py checks every built code object for it: each M0 write is one of these, right
// before its copy, and no instruction the compiler emitted reads M0 (its readers: LDS copies, s_sendmsg, GWS, ds_append
// and ds_consume, LDS-direct / interpolation and s_movrel / v_movrel).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"   // "clobber list contains reserved registers: m0" (intended)
__device__ inline void dma16(__amdgpu_buffer_rsrc_t rsrc, uint32_t lds_base, uint32_t voff, uint32_t soff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :
                 : "s"(lds_base), "v"(voff), "s"(rsrc), "s"(soff)
                 : "memory", "m0");
}

// The same with 4 bytes per lane: lane L's bytes land at lds_base + 4 L.
__device__ inline void dma4(__amdgpu_buffer_rsrc_t rsrc, uint32_t lds_base, uint32_t voff, uint32_t soff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, %3 offen lds"
                 :
                 : "s"(lds_base), "v"(voff), "s"(rsrc), "s"(soff)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

// The copies of one 128-key tile (K and V: 16 KiB each; K scales: 512 B; per-32-key V scales: 512 B) from HBM into
// its LDS ring slots. K and V go by direct copies (buffer_load ... lds, dma below); the 512-thread kernels stage the
// K-scale words through a register (the upper k-group's copy shifted down one byte), the 256-thread kernel copies the
// words directly (dma_ks) and shifts on read. The tile's first key rides in the buffer resource's base and the
// resource's size ends at the sequence's last key, so rows past the end (the last, partial tile) read zeros from the
// range check, and a tile index past the range gets an empty resource (no memory traffic): one branch-free code path.
template <int NT>
struct Stager {
    static constexpr int kN = kTileBytes / (NT * 16);   // 16-byte chunks per thread per 16 KiB tile
    const uint8_t *kb, *vb, *ksb;
    uint32_t ksoff;     // K-scale load offset: key (tid & 127) for tid < 256, out of range (zeros) beyond
    uint32_t kswoff;    // K-scale LDS write offset in a slot (tid < 256: word tid; beyond: the sink)
    uint32_t ksshift;   // 0 for the words (tid < 128), 8 for the shifted copies (128 <= tid < 256)
    uint32_t tid, k_seq, ks_row, SK, lds;
    const uint8_t* vsb; // per-32-key V scales of this (batch, KV head) (extension; unused otherwise)
    uint32_t vs_row;    // bytes between consecutive 32-key blocks of the V-scale tensor (HK 128)

    __device__ void init_vs(const uint8_t* vsb_, uint32_t vs_row_) {
        vsb = uniform_ptr(vsb_);
        vs_row = vs_row_;
    }
    // Resource over the V-scale rows of blocks [blk0, ceil(SK/32)) of this head (empty when `valid` is false or blk0 is
    // past the last block, so such lanes read zeros: E8M0 0, a finite scale for the zero V rows past SK)
    __device__ __forceinline__ __amdgpu_buffer_rsrc_t vs_rsrc(uint32_t blk0, bool valid) const {
        const uint32_t nb = (SK + 31u) >> 5;
        const bool live = valid && blk0 < nb;
        const uint32_t bytes = live ? (nb - 1u - blk0) * vs_row + 128u : 0u;
        return make_rsrc(vsb + (size_t)(live ? blk0 : 0u) * vs_row, bytes);
    }
    // Direct copy of tile [key0, key0 + 128)'s V scales (4 blocks x 128 columns) into V-scale slot `slot`: waves 0 and 1
    // copy two blocks each (lane L: block 2w + L / 32, columns 4 (L % 32) ..); the other waves copy from an empty
    // resource into the sink, so that every wave issues exactly one copy per phase.
    __device__ __forceinline__ void dma_vs(uint32_t key0, bool valid, uint32_t slot) const {
        const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63u;
        const uint32_t dst = w < 2u ? slot_base(lds, kLdsVs, slot, kVsSlot) + 256u * w : lds + kLdsVsSink + 256u * (w - 2u);
        dma4(vs_rsrc((key0 >> 5) + 2u * w, valid && w < 2u), dst, (lane >> 5) * vs_row + 4u * (lane & 31u), 0u);
    }
    // Copy instruction i (0 .. 2 kN - 1: K chunk i / 2 for even i, V chunk i / 2 for odd i) of dma(), alone, so that a
    // wave can spread a tile's copies between its MFMAs instead of waiting for the load path in one burst
    __device__ __forceinline__ void dma_part(int i, uint32_t key0, bool valid, uint32_t slot) const {
        const bool isv = (i & 1) != 0;
        const uint8_t* base = isv ? vb : kb;
        const __amdgpu_buffer_rsrc_t r = make_rsrc(base + (size_t)key0 * k_seq, tile_bytes(key0, valid, k_seq, kD));
        const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);
        const uint32_t dst = slot_base(lds, isv ? kLdsV : kLdsK, slot, kTileBytes);
        const uint32_t g = (uint32_t)(i >> 1) * (NT / 64) + w;
        const uint32_t soff = __builtin_amdgcn_readfirstlane((uint32_t)(i >> 1) * (NT / 8) * k_seq);
        dma16(r, dst + g * 1024u, dmaoff, soff);
    }
    // Direct copy of tile [key0, key0 + 128)'s K-scale words (the words only, no shifted copy: readers use kscale_raw)
    // into K-scale slot `slot`: waves 0 and 1 copy 64 keys each (lane L: key 64 w + L, its 4 bytes at 4 (64 w + L));
    // the other waves copy from an empty resource into the sink, so that every wave issues one copy per tile.
    __device__ __forceinline__ void dma_ks(uint32_t key0, bool valid, uint32_t slot) const {
        const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63u;
        const uint32_t dst = w < 2u ? slot_base(lds, kLdsKs, slot, kKsSlot) + 256u * w : lds + kLdsKsDummy + 256u * ((w - 2u) & 3u);
        const __amdgpu_buffer_rsrc_t r = make_rsrc(ksb + (size_t)key0 * ks_row, tile_bytes(key0, valid && w < 2u, ks_row, 4));
        dma4(r, dst, (64u * (w & 1u) + lane) * ks_row, 0u);
    }

    __device__ void init(const uint8_t* kb_, const uint8_t* vb_, const uint8_t* ksb_, uint32_t k_seq_, uint32_t SK_, uint32_t lds_) {
        // wave-uniform base pointers (readfirstlane states it), so the per-tile resource arithmetic stays scalar
        kb = uniform_ptr(kb_); vb = uniform_ptr(vb_); ksb = uniform_ptr(ksb_);
        tid = threadIdx.x;
        k_seq = k_seq_;
        ks_row = k_seq_ >> 5;
        SK = SK_;
        lds = lds_;
        ksoff = tid < 256u ? (tid & 127u) * ks_row : 0x80000000u;
        kswoff = tid < 256u ? tid * 4u : 0u;
        ksshift = tid < 128u ? 0u : 8u;
    }

    uint32_t ksr;   // the K-scale word of the next tile, loaded in one VALU phase and stored in the next

    // resource size of a tile starting at key0: rem = SK - 1 - key0 keys follow the first, rem stride + tail bytes
    __device__ __forceinline__ uint32_t tile_bytes(uint32_t key0, bool valid, uint32_t stride, int tail) const {
        const int rem = __builtin_amdgcn_readfirstlane((int)SK - 1 - (int)key0);
        return valid ? (uint32_t)max(rem * (int)stride + tail, 0) : 0u;
    }

    // Direct HBM -> LDS copies (buffer_load_dwordx4 ... lds), no VGPR round trip: copy i of wave w writes LDS rows
    // [8 g, 8 g + 8) of the slot, g = i NT/64 + w, lane L the 16 bytes at (8 g + L / 8) 128 + 16 (L & 7), which hold logical
    // chunk (L & 7) ^ swz(row) of that row. Row steps of NT/8 (a multiple of 16) leave swz unchanged, so the lane's
    // source offset is the same for every copy (dmaoff) plus a scalar (i NT/8) rows. A lane past the resource's end
    // gets zeros.
    uint32_t dmaoff;
    __device__ __forceinline__ void init_dma() {
        const uint32_t row = 8u * (tid >> 6) + ((tid & 63u) >> 3);
        dmaoff = row * k_seq + (((tid & 7u) ^ swz(row)) << 4);
    }
    __device__ __forceinline__ void dma(uint32_t kkey0, bool kvalid, uint32_t kslot, uint32_t vkey0, bool vvalid, uint32_t vslot) const {
        const __amdgpu_buffer_rsrc_t rk = make_rsrc(kb + (size_t)kkey0 * k_seq, tile_bytes(kkey0, kvalid, k_seq, kD));
        const __amdgpu_buffer_rsrc_t rv = make_rsrc(vb + (size_t)vkey0 * k_seq, tile_bytes(vkey0, vvalid, k_seq, kD));
        const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);
        const uint32_t kbase = slot_base(lds, kLdsK, kslot, kTileBytes), vbase = slot_base(lds, kLdsV, vslot, kTileBytes);
#pragma unroll
        for (int i = 0; i < kN; ++i) {
            const uint32_t g = (uint32_t)i * (NT / 64) + w;
            const uint32_t soff = __builtin_amdgcn_readfirstlane((uint32_t)i * (NT / 8) * k_seq);
            dma16(rk, kbase + g * 1024u, dmaoff, soff);
            dma16(rv, vbase + g * 1024u, dmaoff, soff);
        }
    }
    // The K-scale words of tile [kkey0, kkey0 + 128) into ksr (register-staged: the upper k-group's copy is shifted)
    __device__ __forceinline__ void load_ks(uint32_t kkey0, bool kvalid) {
        const __amdgpu_buffer_rsrc_t rks = make_rsrc(ksb + (size_t)kkey0 * ks_row, tile_bytes(kkey0, kvalid, ks_row, 4));
        ksr = __builtin_amdgcn_raw_buffer_load_b32(rks, ksoff, 0, 0);
    }
    __device__ __forceinline__ void store_ks(uint32_t kslot) const { store_ks_word(ksr, kslot); }
    // the same through a register the caller holds (the prologue loads several tiles' words at once)
    __device__ __forceinline__ uint32_t ks_word(uint32_t kkey0, bool kvalid) const {
        const __amdgpu_buffer_rsrc_t rks = make_rsrc(ksb + (size_t)kkey0 * ks_row, tile_bytes(kkey0, kvalid, ks_row, 4));
        return __builtin_amdgcn_raw_buffer_load_b32(rks, ksoff, 0, 0);
    }
    __device__ __forceinline__ void store_ks_word(uint32_t word, uint32_t kslot) const {
        const uint32_t ksw_base = tid < 256u ? slot_base(lds, kLdsKs, kslot, kKsSlot) : lds + kLdsKsDummy;
        lds_write4(ksw_base + kswoff, word >> ksshift);
    }

};

// Workgroup barrier that is also a compiler memory barrier (no LDS access moves across it): drains this wave's
// LDS operations (its tile writes become visible) but, unlike __syncthreads, not vmcnt: the staging loads of a
// later tile stay in flight across it.
__device__ inline void block_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// The barrier that publishes the direct HBM -> LDS copies issued one phase earlier: the wave's last M VMEM operations
// (this phase's copies) stay in flight, everything older (vmcnt counts in issue order) has landed in LDS; its LDS
// operations are drained except the last N (the operand reads issued for the next phase).
template <int N, int M>
__device__ inline void block_barrier_keep_dma() {
    static_assert(N >= 0 && N <= 15 && M >= 0 && M <= 63, "waitcnt fields");
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(%1)\n\ts_barrier" ::"n"(M), "n"(N) : "memory");
}

// Softmax recipe constants (softmax.rs:24-27 exact copy; softmax.rs:80-88 lazy copy).
struct Recipe {
    float thr, b131, conv;
    // log2 of the mean ratio of the recipe's exp2 (the pknorm u16 read as bf16, 2^e (1 + m / 128), minus the LUT
    // correction in the exact copy) to 2^x over uniformly distributed fractional parts: 1.037869 (no LUT) and 0.998943
    // (LUT). P/l cancels it in O; the LSE output removes it from log2 l.
    float exp2_bias_log2;
};
// the two recipe copies (softmax.rs:24-27 exact copy with the LUT; softmax.rs:80-88 lazy copy)
__device__ inline Recipe recipe(bool lut) {
    return lut ? Recipe{120.0f / 512.0f, 131.0f / 512.0f, 1.0f, -0.0015262115f}
               : Recipe{__builtin_bit_cast(float, 0x3e85d086u), __builtin_bit_cast(float, 0x3e7df17eu), 0.25f, 0.0536247327f};
}

// Row max of one tile's S^T accumulators: the lane's 64 values (v_max3 chain), then the partner lane l ^ 32
// (the other key half of the same query column) through v_permlane32_swap.
template <int NA>
__device__ __forceinline__ float row_max(const v16f (&s)[NA]) {
    float m = -1.0e30f;
#pragma unroll
    for (int t4 = 0; t4 < NA; ++t4)
#pragma unroll
        for (int i = 0; i < 16; ++i) m = fmaxf(m, s[t4][i]);
    const auto sw = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, m), __builtin_bit_cast(uint32_t, m), false, false);
    return fmaxf(__builtin_bit_cast(float, (uint32_t)sw[0]), __builtin_bit_cast(float, (uint32_t)sw[1]));
}

// The rebase decision of one tile given its row max m: when any lane's max passes the threshold, the new two-word
// reference and the rescale of S, O and the row sums (lanes below the threshold keep their reference, delta = 0).
// (bias: the seed of S, b rm; rm = 1 unless the softmax scale is applied in the kernel)
template <bool LUT, int NA>
__device__ __forceinline__ void rebase(const Recipe& rc, float m, v16f (&s)[NA], v16f (&o)[4], v4f& lacc, float& bias, uint32_t& bw,
                                       float rm) {
    // softmax.rs:125-160 eager: thr < m; softmax.rs:186-241 lazy: !(thr >= m), which also takes NaN
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
        for (int t4 = 0; t4 < NA; ++t4)
#pragma unroll
            for (int i = 0; i < 16; ++i) s[t4][i] += delta;
        const float corr = __builtin_amdgcn_exp2f(delta * 512.0f);
#pragma unroll
        for (int dc = 0; dc < 4; ++dc)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[dc][i] *= corr;
#pragma unroll
        for (int i = 0; i < 4; ++i) lacc[i] *= corr;
        bias = bias_of(bw) * rm;
    }
}

// P = e4m3(pknorm(S') [- LUT] / scale) for one 32-key accumulator: 4 words of 4 keys.
template <bool LUT>
__device__ __forceinline__ void convert_p(const Recipe& rc, const v16f& s, uint32_t (&pw)[4]) {
#pragma unroll
    for (int a = 0; a < 4; ++a) {
        v2u16 u01 = __builtin_bit_cast(v2u16, __builtin_amdgcn_cvt_pknorm_u16(s[4 * a], s[4 * a + 1]));
        v2u16 u23 = __builtin_bit_cast(v2u16, __builtin_amdgcn_cvt_pknorm_u16(s[4 * a + 2], s[4 * a + 3]));
        if (LUT) {
            // u -= LUT[(u >> 4) & 7], LUT = {0, 6, 9, 11, 11, 10, 7, 3} (reduce.rs:84-91)
            const uint32_t i01 = (__builtin_bit_cast(uint32_t, u01) >> 4) & 0x00070007u;
            const uint32_t i23 = (__builtin_bit_cast(uint32_t, u23) >> 4) & 0x00070007u;
            u01 = u01 - __builtin_bit_cast(v2u16, __builtin_amdgcn_perm(0x03070a0bu, 0x0b090600u, i01));
            u23 = u23 - __builtin_bit_cast(v2u16, __builtin_amdgcn_perm(0x03070a0bu, 0x0b090600u, i23));
        }
        // the first conversion writes the low half-word; its "old" operand (whose high half survives until the second
        // conversion overwrites it) is the dead u01 register, so the destination needs no zero-initialisation
        v2s w = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(__builtin_bit_cast(v2s, u01), __builtin_bit_cast(v2bf, u01), rc.conv, false);
        w = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(w, __builtin_bit_cast(v2bf, u23), rc.conv, true);
        pw[a] = __builtin_bit_cast(uint32_t, w);
    }
}

// ---------------------------------------------------------------------------------------------------------------
// One wave's attention over the key range [key_lo, key_hi) of its block: 32 query rows, S^T / O^T in the C layout
// of the 32x32 MFMA (lane = query column n, half hh; value i of accumulator t4 = key 32 t4 + 8 (i / 4) + 4 hh + i % 4).
// ---------------------------------------------------------------------------------------------------------------
template <int NT>
struct Wave {
    static constexpr int ROWS = NT / 64 * 32;
    uint32_t lane, wave, n, hh, lds;
    uint32_t row0;
    int sq[2];
    float vd;
    uint32_t kfo;      // K / Q fragment offset in a tile: row n, chunk (hh ^ swz(n)); chunk 4c + 2e + hh = kfo ^ (4c + 2e) << 4
    uint32_t vfo;      // V^T read offset: row rlo, chunk ((g & 1) ^ swz(rlo)), half pp; dim group dc = vfo ^ (2 dc) << 4
    uint32_t onew;
    uint32_t kso;      // K-scale word offset of this lane: hh 512 + 4 n
    uint32_t vso;      // V-scale byte offset of this lane in a slot: block hh of the 64-key half, column n (+ 32 dc)
    // causal limits: query row i sees keys [0, i + SK - S + 1) (cut to [.., key_hi))
    uint32_t lim_row, lim_wave_min, lim_wave_max, key_hi;
    // softmax state
    uint32_t bw;       // two f16 words (hi = low half); b = 64 makes tile 0 rebase
    float bias;        // the seed of every S accumulator: b of this lane's query (times qrm)
    // the softmax scale applied in the kernel (extension): S' = qm (S + b qrm), the Q scale exponents shifted by qe
    float qm, qrm;
    int32_t qe;
    v16f o[4];
    v4f lacc;
    v4i qtmp[4];       // the lane's Q bytes (32 B of the k-half c = 0 and 32 B of c = 1), resident for the whole range
    uint32_t qsw;      // the lane's Q scale word, loaded by init

    // Q scale operands from the scale word init() loaded (called once the load is likely back)
    __device__ __forceinline__ void commit_q() {
        // Q scale bytes of the two k-halves (E8M0 - 9: S comes out x 2^-9)
#pragma unroll
        for (int c = 0; c < 2; ++c) sq[c] = (int)(((qsw >> (8 * (2 * c + hh))) - 9u + (uint32_t)qe) & 0xffu);
    }

    // Lane constants, softmax state, and the loads of the lane's Q bytes and scales. The Q bytes stay in registers
    // (16 VGPRs) for the whole key range: re-reading them from LDS every tile cost 32 KiB of LDS reads per tile and block.
    // rwave: the wave's 32-row block in the block's rows (its wave index, or wave % 4 when the two groups share rows);
    // rb: query rows per block (ROWS, or 128 for the full-sequence split-tile kernel)
    __device__ __forceinline__ void init(const Prm& p, uint32_t lds_, uint32_t qtile, uint32_t head, uint32_t bidx, uint32_t key_hi_,
                                         uint32_t rwave, uint32_t rb = ROWS) {
        lane = threadIdx.x & 63u;
        wave = wave_id();
        n = lane & 31u;
        hh = lane >> 5;
        lds = lds_;
        key_hi = key_hi_;
        row0 = qtile * rb + rwave * 32u;
        const uint32_t row = row0 + n;
        const uint32_t row_c = min(row, p.S - 1u);
        kfo = n * 128u + ((hh ^ swz(n)) << 4);
        kso = hh * 512u + n * 4u;
        vso = hh * 128u + n;
        {
            const uint8_t* qrow = p.q + (size_t)bidx * p.q_b + (size_t)row_c * p.q_seq + head * kD;
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int e = 0; e < 2; ++e) qtmp[2 * c + e] = *(const GLOBAL_AS v4i*)(qrow + 64 * c + 32 * e + 16 * hh);
        }
        qsw = *(const GLOBAL_AS uint32_t*)(p.qs + (size_t)bidx * p.qs_b + (size_t)row_c * (p.H * 4u) + head * 4u);
        vd = p.vs32 ? 1.0f : *(const GLOBAL_AS float*)p.vd;   // per-32-key V scales ride in the PV MFMAs instead
        lim_row = lim_wave_min = lim_wave_max = key_hi;
        if (p.flags & 1u) {
            const int off = (int)p.SK - (int)p.S + 1;
            lim_row = (uint32_t)max(0, min((int)key_hi, (int)row + off));
            lim_wave_min = (uint32_t)max(0, min((int)key_hi, (int)row0 + off));
            lim_wave_max = (uint32_t)max(0, min((int)key_hi, (int)row0 + 31 + off));
        }
        {
            // ds_read_b64_tr_b8 source lane (g, jj, pp) reads key 16 r + rlo of the 64-key half, dims
            // 32 dc + 16 (g & 1) + 8 pp .. +7
            const uint32_t g = lane >> 4, jj = (lane >> 1) & 7u, pp = lane & 1u;
            const uint32_t rlo = 8u * (jj >> 2) + 4u * (g >> 1) + (jj & 3u);
            vfo = rlo * 128u + (((g & 1u) ^ swz(rlo)) << 4) + 8u * pp;
        }
        // ones pattern of the row-sum MFMA (16x16x128): lane la holds A row la % 16, k-groups la / 16; row m sums
        // the P bytes of query (m % 2 ? n + 16 : n) -> ones iff (la / 16) % 2 == la % 2
        onew = (((lane >> 4) & 1u) == (lane & 1u)) ? 0x38383838u : 0u;
        qm = p.qk_m;
        qrm = p.qk_rm;
        qe = p.qk_e;
        bw = 0x48004800u;
        bias = bias_of(bw) * qrm;
#pragma unroll
        for (int dc = 0; dc < 4; ++dc)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[dc][i] = 0.0f;
        lacc = (v4f){0.0f, 0.0f, 0.0f, 0.0f};
    }

    __device__ __forceinline__ bool active(uint32_t key0) const { return key0 < lim_wave_max; }
    __device__ __forceinline__ bool needs_mask(uint32_t key0) const { return key0 + kTile > min(key_hi, lim_wave_min); }
    // S' = qm S_acc (S_acc seeded with b qrm) when the softmax scale is applied in the kernel; a row max taken before
    // scales the same way (qm > 0 and rounding are monotonic).
    template <int NA>
    __device__ __forceinline__ void scale_s(v16f (&s)[NA], float& m) const {
#pragma unroll
        for (int t4 = 0; t4 < NA; ++t4)
#pragma unroll
            for (int i = 0; i < 16; ++i) s[t4][i] *= qm;
        m *= qm;
    }
    // keys at or past the range end / causal limit: -1e30 takes no part in the max and converts to P = 0 (pknorm
    // clamps), the reference's two fills (reduce.rs:13-49) in one
    // (accumulator a holds 32-key block KB0 + a of the tile)
    template <int KB0 = 0, int NA>
    __device__ __forceinline__ void apply_mask(v16f (&s)[NA], uint32_t key0) const {
        const int nvalid = (int)min(key_hi, lim_row) - (int)key0 - 4 * (int)hh;
#pragma unroll
        for (int t4 = 0; t4 < NA; ++t4)
#pragma unroll
            for (int i = 0; i < 16; ++i) s[t4][i] = (32 * (KB0 + t4) + 8 * (i >> 2) + (i & 3)) < nvalid ? s[t4][i] : -1.0e30f;
    }

    // 32-byte K or Q fragment of k-half c (c = 0: d 0..63, 1: d 64..127) of row n of the tile at `base`
    // (The slot base is added to the lane offset first and the 4 KiB block offset last, so the block offset folds into
    // the instruction's immediate: one address add per lane-offset variant and tile instead of one per read.)
    __device__ __forceinline__ v8i frag(uint32_t base, int c, uint32_t block_off = 0) const {
        return cat8(lds_read16(lane_addr(base, kfo ^ ((uint32_t)(4 * c) << 4)) + block_off),
                    lds_read16(lane_addr(base, kfo ^ ((uint32_t)(4 * c + 2) << 4)) + block_off));
    }
    // the lane's Q bytes stay in registers: fragment c = bytes [64 c + 16 hh, +16) and [64 c + 32 + 16 hh, +16) of its row
    __device__ __forceinline__ v8i qfrag(int c) const { return cat8(qtmp[2 * c], qtmp[2 * c + 1]); }
    // K-scale word of 32-key block t4 for this lane's key row, read from the copy shifted down by hh bytes so that
    // op_sel byte 2c is the lane half's E8M0 byte 2c + hh
    __device__ __forceinline__ uint32_t kscale(uint32_t ksb, int t4) const { return lds_read4(lane_addr(ksb, kso) + 128u * t4); }
    // The same from a slot that holds the words only (copied straight from HBM): the upper lane half shifts its word
    // down one byte itself
    __device__ __forceinline__ uint32_t kscale_raw(uint32_t ksb, int t4) const {
        return lds_read4(lane_addr(ksb, 4u * n) + 128u * t4) >> (8u * hh);
    }
    // E8M0 of PV MFMA (j, dc)'s k-block for this lane: in the scaled MFMA, lane r + 32 kb supplies the scale of row r
    // (column 32 dc + n) over k-block kb, which is 32-key block 2 j + kb of the tile (the S^T tile the P bytes came from)
    __device__ __forceinline__ uint32_t vscale(uint32_t vsb, int j, int dc) const {
        return *(const LDS_AS uint8_t*)(uintptr_t)(lane_addr(vsb, vso) + 256u * j + 32u * dc);
    }
    // V^T fragment of PV MFMA (j, dc): four transposing reads 16 keys apart
    __device__ __forceinline__ v8i vfrag(uint32_t vb, int j, int dc) const {
        const uint32_t va = lane_addr(vb, vfo ^ ((uint32_t)(2 * dc) << 4)) + 8192u * j;
        const v2i r0 = lds_read_tr8(va), r1 = lds_read_tr8(va + 2048u), r2 = lds_read_tr8(va + 4096u), r3 = lds_read_tr8(va + 6144u);
        return (v8i){r0[0], r0[1], r1[0], r1[1], r2[0], r2[1], r3[0], r3[1]};
    }
    template <int NA>
    __device__ __forceinline__ static v8i pfrag(const uint32_t (&pw)[NA][4], int j) {
        return (v8i){(int)pw[2 * j][0], (int)pw[2 * j][1], (int)pw[2 * j][2], (int)pw[2 * j][3],
                     (int)pw[2 * j + 1][0], (int)pw[2 * j + 1][1], (int)pw[2 * j + 1][2], (int)pw[2 * j + 1][3]};
    }
    // The ones operand of the row-sum MFMA, rebuilt where it is used (an opaque copy, so the compiler neither keeps
    // it live across the loop nor hoists it: 8 VGPRs only around the row-sum MFMAs).
    __device__ __forceinline__ v8i ones_op() const {
        uint32_t x = onew;
        asm volatile("" : "+v"(x));   // a copy the compiler makes (and hazard-checks), as in lane_addr
        return __builtin_bit_cast(v8i, splat8(__builtin_bit_cast(float, x)));
    }
    __device__ __forceinline__ v16f qk_mfma(const v8i& kf, const v8i& qf, const v16f& c_in, uint32_t ksw, int c) const {
        // scaled fp8 MFMA: A = K (rows = keys), B = Q^T (columns = queries), E8M0 scales per 32 of k
        return c == 0 ? __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(kf, qf, c_in, 0, 0, 0, (int)ksw, 0, sq[0])
                      : __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(kf, qf, c_in, 0, 0, 2, (int)ksw, 0, sq[1]);
    }

    // S(t+1): k-half 0 of all four 32-key accumulators, then k-half 1 (one Q fragment live at a time). The seed
    // (16 copies of b) is written into s[3] and is the C input of the first MFMA of s[0..2]; s[3] then accumulates
    // in place: no separate seed registers. One K fragment is read one MFMA ahead.
    // (NA accumulators: 32-key blocks KB0 .. KB0 + NA - 1 of the tile)
    template <int KB0 = 0, int NA, bool RAWKS = false>
    __device__ __forceinline__ void qk_all(uint32_t nslot, v16f (&s)[NA]) {
#pragma unroll
        for (int i = 0; i < 16; ++i) s[NA - 1][i] = bias;
        const uint32_t kb = slot_base(lds, kLdsK, nslot, kTileBytes);
        const uint32_t ksb = slot_base(lds, kLdsKs, nslot, (uint32_t)kKsSlot);
        auto kread = [&](int g) { return frag(kb, g / NA, 4096u * (uint32_t)(KB0 + g % NA)); };   // g = NA c + t4
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const v8i qf = qfrag(c);
            v8i kc = kread(NA * c);
#pragma unroll
            for (int t4 = 0; t4 < NA; ++t4) {
                const int g = NA * c + t4;
                v8i kn = kc;
                if (g < 2 * NA - 1) kn = kread(g + 1);
                const uint32_t ksw = RAWKS ? kscale_raw(ksb, KB0 + t4) : kscale(ksb, KB0 + t4);
                s[t4] = qk_mfma(kc, qf, c == 0 ? s[NA - 1] : s[t4], ksw, c);
                kc = kn;
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }

    static constexpr int DEPTH = FMHA_PREFETCH;   // MFMA-phase operand reads run DEPTH MFMAs ahead
    typedef v8i Ring[DEPTH + 1];

    // The MFMA phase with QK(t+1) first (i = 0..7: k-half c = i / 4, accumulator t4 = i % 4) and PV(t) second (i = 8..15:
    // V^T fragment (j, dc) = ((i - 8) / 4, (i - 8) % 4), row sums at dc = 0), so that S(t+1) is complete while PV(t)
    // runs: the row max of S(t+1) (a quarter behind each of the first PV MFMAs) moves out of the VALU phase into the
    // MFMA shadow. It is the unmasked maximum: a tile that needs the causal/tail mask is masked, and its maximum
    // taken again, in its VALU phase (a masked write of S here, under the MFMAs, made the register allocation spill). Operands are read DEPTH MFMAs ahead across the QK -> PV seam; the first
    // DEPTH K fragments, the Q fragment of k-half 0 and the K-scale words come from qk_prefetch. Returns the row max.
    struct QkPre {
        v8i qf0;
        uint32_t ksw[4];
    };
    template <int NA = 4, int KB0 = 0>
    __device__ __forceinline__ void qk_prefetch(uint32_t kslot, Ring& ring, QkPre& pre) const {
        static_assert(DEPTH <= 2 * NA, "the prefetched operands are K fragments");
        const uint32_t kb = slot_base(lds, kLdsK, kslot, kTileBytes);
        const uint32_t ksb = slot_base(lds, kLdsKs, kslot, (uint32_t)kKsSlot);
#pragma unroll
        for (int i = 0; i < DEPTH; ++i) ring[i] = frag(kb, i / NA, 4096u * (uint32_t)(KB0 + i % NA));
        pre.qf0 = qfrag(0);
#pragma unroll
        for (int t4 = 0; t4 < NA; ++t4) pre.ksw[t4] = kscale(ksb, KB0 + t4);
    }

    // NA < 4: the wave's keys are the tile's 32-key blocks KB0 .. KB0 + NA - 1 (NA = 2: one 64-key half; 2 NA QK and
    // 2 NA PV MFMAs, indices shifted accordingly).
    template <bool QK, bool VS = false, int KB0 = 0, int NA = 4>
    __device__ __forceinline__ float m_phase_qf(uint32_t vslot, const uint32_t (&pw)[NA][4], uint32_t kslot, v16f (&s)[NA], Ring& ring,
                                                const QkPre& pre) {
        constexpr int NQ = 2 * NA, NI = 4 * NA;   // QK MFMAs, all MFMAs
        const uint32_t vb = slot_base(lds, kLdsV, vslot, kTileBytes);
        uint32_t vsc[2 * NA];   // per-32-key V scales of the PV MFMAs (extension), read a few MFMAs ahead of PV
        auto read_vs = [&] {
            const uint32_t vsb = slot_base(lds, kLdsVs, vslot, kVsSlot);
#pragma unroll
            for (int g = 0; g < 2 * NA; ++g) vsc[g] = vscale(vsb, KB0 / 2 + (g >> 2), g & 3);
        };
        const uint32_t kb = slot_base(lds, kLdsK, kslot, kTileBytes);
        constexpr int I0 = QK ? 0 : NQ;
        auto fetch = [&](int i) -> v8i {
            return i < NQ ? frag(kb, i / NA, 4096u * (uint32_t)(KB0 + i % NA)) : vfrag(vb, KB0 / 2 + ((i - NQ) >> 2), (i - NQ) & 3);
        };
        v8i qf1;
        v8i ones;
        float mx = -1.0e30f;
        // The row max of S(t+1) in eighths behind the PV MFMAs (four accumulators: the 256-row blocks; the last eighth
        // after the last MFMA) rather than in quarters behind the first four: fewer VALU instructions between two MFMAs
        // of this wave, which the other wave's conversions hold up (cfg2 -0.6 %, cfg3 -0.4 %; the split-tile blocks'
        // two accumulators keep the quarters, +3 % at cfg4 in eighths).
        constexpr bool kSpread = NA == 4;
        if (!QK) {
#pragma unroll
            for (int i = I0; i < I0 + DEPTH; ++i) ring[i % (DEPTH + 1)] = fetch(i);
            ones = ones_op();
            if (VS) read_vs();
        }
#pragma unroll
        for (int i = I0; i < NI; ++i) {
            if (i + DEPTH < NI) ring[(i + DEPTH) % (DEPTH + 1)] = fetch(i + DEPTH);
            if (QK && i == NA - 2) qf1 = qfrag(1);
            if (QK && i == NQ - 3) ones = ones_op();
            if (VS && QK && i == NQ - 4) read_vs();
            __builtin_amdgcn_sched_barrier(0);
            if (i < NQ) {
                const int c = i / NA, t4 = i % NA;
                s[t4] = qk_mfma(ring[i % (DEPTH + 1)], c == 0 ? pre.qf0 : qf1, c == 0 ? s[NA - 1] : s[t4], pre.ksw[t4], c);
            } else {
                const int j = (i - NQ) >> 2, dc = (i - NQ) & 3;
                const v8i pf = pfrag(pw, j);
                if (dc == 0) lacc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(ones, pf, lacc, 0, 0, 0, 127, 0, 127);
                o[dc] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(ring[i % (DEPTH + 1)], pf, o[dc], 0, 0, 0,
                                                                         VS ? (int)vsc[i - NQ] : 127, 0, 127);
            }
            __builtin_amdgcn_sched_barrier(0);
            // row max of S(t+1): accumulator a behind PV MFMA NQ + 1 + a (accumulator a's last QK MFMA is i = NA + a)
            if (QK && !kSpread && i >= NQ + 1 && i <= NQ + NA) {
#pragma unroll
                for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[i - NQ - 1][e]);
                asm volatile("" : "+v"(mx));   // pins this quarter here (the reduction would otherwise sink past the MFMAs)
            }
            if (QK && kSpread && i >= NQ + 1 && i <= NQ + 2 * NA - 1) {
                const int j = i - NQ - 1;   // half-accumulator j: 8 values behind PV MFMA NQ + 1 + j, the last after the loop
#pragma unroll
                for (int e = 0; e < 8; ++e) mx = fmaxf(mx, s[j >> 1][8 * (j & 1) + e]);
                asm volatile("" : "+v"(mx));
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if (QK && kSpread) {
#pragma unroll
            for (int e = 0; e < 8; ++e) mx = fmaxf(mx, s[NA - 1][8 + e]);
        }
        if (!QK) return 0.0f;
        const auto sw = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, mx), __builtin_bit_cast(uint32_t, mx), false, false);
        return fmaxf(__builtin_bit_cast(float, (uint32_t)sw[0]), __builtin_bit_cast(float, (uint32_t)sw[1]));
    }

    // The MFMA phase of a wave that has its SIMD to itself (the 256-thread block): no second wave converts under its
    // MFMAs, so it does its own VALU work between them. QK(t+1) (8 MFMAs, into sn, seeded with the bias) runs with the
    // conversion of S(t) (sc, already rebased) to P(t), one 32-key accumulator after every second MFMA; PV(t) (8 MFMAs
    // and the 2 row-sum MFMAs) runs with the unmasked row max of S(t+1), as in m_phase_qf. Without QK (the last tile)
    // the conversion comes first. after_mfma(i) runs behind MFMA i (the caller's tile copies: issued in one burst, they
    // held the wave ~1,100 cycles per tile at the load path). Operands are read DEPTH MFMAs ahead across the seam,
    // inside the phase (reading the first ones behind the previous barrier, under the rebase, was slower). Measured
    // alternatives that were no faster: half of the conversion moved under the PV MFMAs; copies from MFMA 6 on.
    // Returns the row max.
    template <bool LUT, bool VS, bool QK, typename F>
    __device__ __forceinline__ float m_phase_cv(const Recipe& rc, uint32_t vslot, uint32_t kslot, v16f (&sc)[4], v16f (&sn)[4],
                                                uint32_t (&pw)[4][4], const F& after_mfma) {
        constexpr int NQ = QK ? 8 : 0, NI = NQ + 8;
        const uint32_t vb = slot_base(lds, kLdsV, vslot, kTileBytes);
        const uint32_t kb = slot_base(lds, kLdsK, kslot, kTileBytes);
        auto fetch = [&](int i) -> v8i {
            return i < NQ ? frag(kb, i / 4, 4096u * (uint32_t)(i % 4)) : vfrag(vb, (i - NQ) >> 2, (i - NQ) & 3);
        };
        Ring ring;
#pragma unroll
        for (int i = 0; i < DEPTH; ++i) ring[i] = fetch(i);
        uint32_t ksw[4];
        v8i qf;
        if (QK) {
            const uint32_t ksb = slot_base(lds, kLdsKs, kslot, (uint32_t)kKsSlot);
#pragma unroll
            for (int t4 = 0; t4 < 4; ++t4) ksw[t4] = kscale_raw(ksb, t4);
            qf = qfrag(0);
            sn[3] = splat16(bias);
        } else {
#pragma unroll
            for (int t4 = 0; t4 < 4; ++t4) convert_p<LUT>(rc, sc[t4], pw[t4]);
        }
        uint32_t vsc[8];
        if (VS) {
            const uint32_t vsb = slot_base(lds, kLdsVs, vslot, kVsSlot);
#pragma unroll
            for (int g = 0; g < 8; ++g) vsc[g] = vscale(vsb, g >> 2, g & 3);
        }
        const v8i ones = ones_op();
        float mx = -1.0e30f;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            if (i + DEPTH < NI) ring[(i + DEPTH) % (DEPTH + 1)] = fetch(i + DEPTH);
            if (QK && i == 4) qf = qfrag(1);
            __builtin_amdgcn_sched_barrier(0);
            if (i < NQ) {
                const int c = i / 4, t4 = i % 4;
                sn[t4] = qk_mfma(ring[i % (DEPTH + 1)], qf, c == 0 ? sn[3] : sn[t4], ksw[t4], c);
            } else {
                const int j = (i - NQ) >> 2, dc = (i - NQ) & 3;
                const v8i pf = pfrag(pw, j);
                if (dc == 0) lacc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(ones, pf, lacc, 0, 0, 0, 127, 0, 127);
                o[dc] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(ring[i % (DEPTH + 1)], pf, o[dc], 0, 0, 0,
                                                                         VS ? (int)vsc[i - NQ] : 127, 0, 127);
            }
            __builtin_amdgcn_sched_barrier(0);
            after_mfma(i);
            if (QK && i < NQ && (i & 1) == 0) convert_p<LUT>(rc, sc[i >> 1], pw[i >> 1]);
            // row max of S(t+1), half an accumulator at a time: half j behind PV MFMA NQ + 1 + j (accumulator j / 2's last
            // QK MFMA is i = 4 + j / 2)
            // (eighths behind the PV MFMAs, the last after them, rather than quarters behind the first four: the
            // published t128 shapes -0.5 %, cfg1 -1.5 %)
            if (QK && i >= NQ + 1 && i <= NQ + 7) {
                const int j = i - NQ - 1;
#pragma unroll
                for (int e = 0; e < 8; ++e) mx = fmaxf(mx, sn[j >> 1][8 * (j & 1) + e]);
                asm volatile("" : "+v"(mx));
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if (QK) {
#pragma unroll
            for (int e = 0; e < 8; ++e) mx = fmaxf(mx, sn[3][8 + e]);
        }
        if (!QK) return 0.0f;
        const auto sw = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, mx), __builtin_bit_cast(uint32_t, mx), false, false);
        return fmaxf(__builtin_bit_cast(float, (uint32_t)sw[0]), __builtin_bit_cast(float, (uint32_t)sw[1]));
    }

};

// The row sum of this lane's query (the ones pattern puts it in D dword (lane / 16) % 2).
__device__ __forceinline__ float row_sum(const v4f& lacc, uint32_t lane) { return ((lane >> 4) & 1u) ? lacc[1] : lacc[0]; }

// The running state of the LSE-weighted merge (epilogue.rs:89-167) for 8 outputs of one row: base-2 maximum, weight
// sum and the weighted sums.
struct MergeState {
    float m, den, acc[8];
};

__device__ __forceinline__ void merge_init(MergeState& st) {
    st.m = -1.0e30f;
    st.den = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) st.acc[i] = 0.0f;
}

// st <- st merged with the splits lo .. hi - 1 (lo < hi), in order, for group t: outputs 8 (t & 15) .. +7 of partial
// row t >> 4. F32: f32 partial rows (the extension) instead of fp16. The splits go in chunks of 8: every load of a
// chunk is issued before its first merge step, in one straight-line block with no branch, so a chunk costs one memory
// latency (with a branch per split on the row format, the compiler waited for each split's loads in turn).
template <bool F32>
__device__ __forceinline__ void merge_splits(const float* lse, const uint8_t* ohat, uint32_t rows, uint32_t lo, uint32_t hi,
                                             uint32_t t, MergeState& st) {
    constexpr int NW = F32 ? 8 : 4;      // dwords of one split's 8 values
    // byte offsets below 2^32: validate refuses split partials of 4 GiB or more
    const __amdgpu_buffer_rsrc_t rl = make_rsrc(lse, 0xffffffffu), ro = make_rsrc(ohat, 0xffffffffu);
    auto load = [&](uint32_t s, uint32_t& l, uint32_t (&xw)[NW]) {
        const uint32_t r = s * rows + (t >> 4);   // partial row index
        l = __builtin_amdgcn_raw_buffer_load_b32(rl, r * 4u, 0, 0);
        const uint32_t off = ((r << 4) | (t & 15u)) * (F32 ? 32u : 16u);
        const v4i x0 = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(ro, off, 0, 0));
#pragma unroll
        for (int i = 0; i < 4; ++i) xw[i] = (uint32_t)x0[i];
        if (F32) {
            const v4i x1 = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(ro, off + 16u, 0, 0));
#pragma unroll
            for (int i = 0; i < NW - 4; ++i) xw[4 + i] = (uint32_t)x1[i];
        }
    };
    auto merge = [](MergeState& st, float l, const uint32_t (&xw)[NW]) {
        float x[8];
#pragma unroll
        for (int i = 0; i < NW; ++i) {
            if (F32) x[i] = __builtin_bit_cast(float, xw[i]);
            else { x[2 * i] = h2f(xw[i]); x[2 * i + 1] = h2f(xw[i] >> 16); }
        }
        const float m_new = fmaxf(st.m, l);
        const float dm = m_new * -1.0f;
        const float al = __builtin_amdgcn_exp2f(st.m + dm);
        const float w = __builtin_amdgcn_exp2f(l + dm);
        st.den = st.den * al + w;
#pragma unroll
        for (int i = 0; i < 8; ++i) st.acc[i] = st.acc[i] * al + w * x[i];
        st.m = m_new;
    };
    // indices past hi re-read split hi - 1, which is not merged again
    for (uint32_t s0 = lo; s0 < hi; s0 += 8u) {
        uint32_t l[8], xw[8][NW];
#pragma unroll
        for (uint32_t s = 0; s < 8u; ++s) load(min(s0 + s, hi - 1u), l[s], xw[s]);
#pragma unroll
        for (uint32_t s = 0; s < 8u; ++s)
            if (s0 + s < hi) merge(st, __builtin_bit_cast(float, l[s]), xw[s]);
    }
}

// a <- a merged with b (b covering splits after a's): the same weighting as one split's step, with b's weight sum and
// weighted sums in place of one split's 1 and values.
__device__ __forceinline__ void merge_states(MergeState& a, const MergeState& b) {
    const float m_new = fmaxf(a.m, b.m);
    const float dm = m_new * -1.0f;
    const float al = __builtin_amdgcn_exp2f(a.m + dm);
    const float w = __builtin_amdgcn_exp2f(b.m + dm);
    a.den = a.den * al + b.den * w;
#pragma unroll
    for (int i = 0; i < 8; ++i) a.acc[i] = a.acc[i] * al + b.acc[i] * w;
    a.m = m_new;
}

// the 8 bf16 results acc / den
__device__ __forceinline__ v4i merge_finish(const MergeState& st) {
    const float rd = __builtin_amdgcn_rcpf(st.den);
    v4i out;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const v2bf w = {(__bf16)(st.acc[2 * i] * rd), (__bf16)(st.acc[2 * i + 1] * rd)};
        out[i] = __builtin_bit_cast(int, w);
    }
    return out;
}

// Epilogue. Full-sequence kernels: O = O^T . (v_descale / l) -> bf16 rows (state.rs:79-83); the optional natural-log
// LSE. KV split: the fp16 partial O-hat = (O / 16) (v_descale / l_total) with l_total = l / 16 and
// lse = log2(l_total) - 2048 (hi + lo) (block3.rs:291-356, softmax.rs:308-322), partial row
// split * rows_total + (b S + row) H + h. A row with no visible key (causal, S > SK) writes zeros.
// The 16-bit rows go through LDS: each lane holds 4-dim pieces of one row (the MFMA C layout), so direct stores would
// touch 32 rows (32 cache lines) per instruction; staged as [32 rows][256 B] per wave, 16 lanes write one row's 256 B
// with 16-byte stores. `sync`: the ring may still be read by other waves (a block barrier first). TAIL (the ping-pong
// kernels' group B, which ends its loop one MFMA phase before group A): the rows go through the wave's own slot past
// the ring in two rounds of 16 rows, without waiting for A, and B's block barrier, which pairs with the one A takes
// before staging over the ring, comes after B's stores are issued. (The 256-thread kernel's waves end together:
// there the two rounds cost more than the barrier saves.) DCH: the dims the wave writes: 0 all, 1 dims 0..63 (dc 0, 1),
// 2 dims 64..127 (dc 2, 3; the LSE is left to the DCH 1 wave of the same rows).
template <bool SPLIT, int NT, bool TAIL = false, int DCH = 0>
__device__ __forceinline__ void epilogue(const Prm& p, const Wave<NT>& w, uint32_t head, uint32_t bidx, uint32_t split, const Recipe& rc,
                                         bool sync) {
    // lane-derived values recomputed here from an opaque lane id: kept from the prologue they would be live (and
    // spilled) across the whole loop
    uint32_t all = ~0u;
    asm volatile("" : "+s"(all));   // an opaque mask, so the lane index is computed here (see lane_addr on inline asm)
    const uint32_t lane = __builtin_amdgcn_mbcnt_hi(all, __builtin_amdgcn_mbcnt_lo(all, 0u));
    const uint32_t hh = lane >> 5, n = lane & 31u, row = w.row0 + n;
    const float l = row_sum(w.lacc, lane);
    const uint32_t dbase = 4u * hh;
    const bool f32 = SPLIT && p.f32_partials;
    constexpr int kDc0 = DCH == 2 ? 2 : 0, kDc1 = DCH == 1 ? 2 : 4;   // the dc range written
    static_assert(!(TAIL && DCH != 0), "the tail staging writes whole rows");
    // per-lane factor and 16-bit conversion of the row pieces
    float fin;
    if (!SPLIT) {
        fin = l > 0.0f ? __builtin_amdgcn_rcpf(l) * w.vd : 0.0f;
    } else {
        const float l_total = l * 0.0625f;
        fin = l > 0.0f ? __builtin_amdgcn_rcpf(l_total) * w.vd : 0.0f;
    }
    // base of row 0 of this wave's 32 rows and the row stride (bytes), wave-uniform
    uint8_t* obase;
    size_t ostride;
    if (!SPLIT) {
        obase = p.o + (size_t)bidx * p.o_b + head * 256u + (size_t)w.row0 * p.o_seq;
        ostride = p.o_seq;
    } else {
        const size_t prow0 = (size_t)split * p.rows_total + ((size_t)bidx * p.S + w.row0) * p.H + head;
        obase = p.ohat + prow0 * (f32 ? 512u : 256u);
        ostride = (size_t)p.H * (f32 ? 512u : 256u);
    }
    if (f32) {
        // extension: f32 rows of 512 B (the workspace's rows are fp32-sized either way), stored directly
        if (row < p.S) {
            uint8_t* orow = obase + (size_t)n * ostride;
#pragma unroll
            for (int dc = kDc0; dc < kDc1; ++dc)
#pragma unroll
                for (int a = 0; a < 4; ++a) {
                    v4f x;
#pragma unroll
                    for (int e = 0; e < 4; ++e) x[e] = (w.o[dc][4 * a + e] * 0.0625f) * fin;
                    *(v4f*)(orow + (32 * dc + 8 * a + dbase) * 4) = x;
                }
        }
    } else {
        if (sync && !TAIL) block_barrier();
        const float fin16 = fin * 0.0625f;   // (x / 16) fin == x (fin / 16) exactly: 1/16 is a power of two
        // the row's 16-bit words: wd[dc][a][c] holds dims 32 dc + 8 a + dbase + 2 c and + 1
        uint32_t wd[4][4][2];
#pragma unroll
        for (int dc = kDc0; dc < kDc1; ++dc)
#pragma unroll
            for (int a = 0; a < 4; ++a)
#pragma unroll
                for (int c = 0; c < 2; ++c) {
                    const float x0 = w.o[dc][4 * a + 2 * c], x1 = w.o[dc][4 * a + 2 * c + 1];
                    if (!SPLIT) {
                        const v2bf b = {(__bf16)(x0 * fin), (__bf16)(x1 * fin)};
                        wd[dc][a][c] = __builtin_bit_cast(uint32_t, b);
                    } else {
                        // the f32 products are rounded, then converted to f16 (RNE): the empty asm keeps the compiler
                        // from fusing product and conversion into one rounding (v_fma_mix), which differs in
                        // double-rounding cases; v_cvt_pk_f16_f32 converts the pair
                        float y0 = x0 * fin16, y1 = x1 * fin16;
                        asm volatile("" : "+v"(y0), "+v"(y1));
                        wd[dc][a][c] = __builtin_bit_cast(uint32_t, __builtin_convertvector((v2f){y0, y1}, v2h));
                    }
                }
        const uint32_t c16 = lane & 15u;
        if (!TAIL) {
            const uint32_t sbase = w.lds + kLdsEpi + wave_id() * 32u * kEpiRow;
#pragma unroll
            for (int dc = kDc0; dc < kDc1; ++dc)
#pragma unroll
                for (int a = 0; a < 4; ++a)
                    *(LDS_AS v2i*)(uintptr_t)(sbase + n * kEpiRow + (32 * dc + 8 * a + dbase) * 2) = (v2i){(int)wd[dc][a][0], (int)wd[dc][a][1]};
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // the wave reads back only its own rows
            if (DCH == 0) {
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const uint32_t r = 4u * k + (lane >> 4);
                    const v4i x = lds_read16(sbase + r * kEpiRow + c16 * 16u);
                    if (w.row0 + r < p.S) {
                        store16_system(obase + (size_t)r * ostride + c16 * 16u, x);
                    }
                }
            } else {
                // half rows: 8 lanes store one row's 128 B
                const uint32_t c8 = (lane & 7u) + (DCH == 2 ? 8u : 0u);
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const uint32_t r = 8u * k + (lane >> 3);
                    const v4i x = lds_read16(sbase + r * kEpiRow + c8 * 16u);
                    if (w.row0 + r < p.S) {
                        store16_system(obase + (size_t)r * ostride + c8 * 16u, x);
                    }
                }
            }
        } else {
            // rows 16 h .. 16 h + 15 per round (the lanes of those rows write, every lane reads back and stores)
            const uint32_t sbase = w.lds + kLdsTail + (wave_id() & 3u) * 16u * kEpiRow;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                if ((n >> 4) == (uint32_t)h) {
#pragma unroll
                    for (int dc = 0; dc < 4; ++dc)
#pragma unroll
                        for (int a = 0; a < 4; ++a)
                            *(LDS_AS v2i*)(uintptr_t)(sbase + (n & 15u) * kEpiRow + (32 * dc + 8 * a + dbase) * 2) =
                                (v2i){(int)wd[dc][a][0], (int)wd[dc][a][1]};
                }
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const uint32_t r = 4u * k + (lane >> 4);
                    const v4i x = lds_read16(sbase + r * kEpiRow + c16 * 16u);
                    if (w.row0 + 16u * h + r < p.S) {
                        store16_system(obase + (size_t)(16u * h + r) * ostride + c16 * 16u, x);
                    }
                }
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // round h's reads are back before h + 1 writes
            }
            if (sync) block_barrier();   // pairs with A's barrier before its staging
        }
    }
    if (row >= p.S || hh != 0 || DCH == 2) return;
    if (!SPLIT) {
        if (p.lse_out) {
            // natural-log LSE of the scores (extension): P = 2^(S + 512 b - 127) / conv, l = sum P
            const float hl = h2f(w.bw) + h2f(w.bw >> 16);
            const float lse2 = l > 0.0f ? __builtin_amdgcn_logf(l) - hl * 2048.0f + 127.0f + __builtin_amdgcn_logf(rc.conv) - rc.exp2_bias_log2
                                        : -INFINITY;
            store4_system(p.lse_out + ((size_t)bidx * p.H + head) * p.S + row, lse2 * 0.69314718055994531f);
        }
    } else {
        const float l_total = l * 0.0625f;
        const float hl = h2f(w.bw) + h2f(w.bw >> 16);
        const size_t prow = (size_t)split * p.rows_total + ((size_t)bidx * p.S + row) * p.H + head;
        // an empty range (l = 0) gets -1e30: the combine gives it weight 0
        // a write-back store: the H words of a row are consecutive, and the KV split's one-query-tile grids put the
        // blocks of those H heads on one XCD (kvsplit_kernel), so its L2 merges them into whole lines (written through,
        // each 4-byte word cost a 32-byte memory write)
        *(GLOBAL_AS float*)(p.lse + prow) = l > 0.0f ? __builtin_amdgcn_logf(l_total) + (hl * 2048.0f) * -1.0f : -1.0e30f;
    }
}

// The two key halves of one row block (HV): wave w of group A (waves 0-3) and wave w + 4 of group B hold the same 32
// rows in the same lane layout, each with the softmax state of its half of every tile's keys. Each hands the other
// the O values of the dims the other finishes: B gives A dims 0..63 (O groups dc 0, 1), A gives B dims 64..127
// (dc 2, 3), as 8 four-value groups, 16 bytes per lane and group, lane-contiguous, over the dead K/V ring, with its
// row sum and bias word. With b the stream's bias (O and l carry a factor 2^(512 b)), the smaller b is kept and the
// other stream is scaled by 2^(512 (b_min - b)) <= 1; an empty stream (b = 64, O = l = 0) adds zeros. Both groups
// evaluate the same expressions on the same operands (A's stream times sa, B's times sb, B's added by the fma), so
// the merged row sum and bias word agree bit for bit and each group writes its half of every row. Every wave of the
// block calls it (two block barriers).
// (Whole v4 groups: stores of single elements extracted from the accumulators were merged by the compiler into
// ds_write2st64 pairs that repeated one element.)
template <bool GB, int NT>
__device__ __forceinline__ void merge_halves(Wave<NT>& w, uint32_t lds) {
    constexpr uint32_t kGroups = 17u;   // B -> A groups 0..7, A -> B groups 8..15, then (l_a, bw_a, l_b, bw_b)
    constexpr int kGive = GB ? 0 : 2;   // the dc pair this group hands over
    constexpr int kKeep = GB ? 2 : 0;   // the dc pair it finishes
    block_barrier();                    // every wave is done with the ring (its copies drained before)
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t base = lds + kLdsK + (wave_id() & 3u) * kGroups * 1024u + lane * 16u;
    const float l_own = row_sum(w.lacc, lane);
#pragma unroll
    for (int g = 0; g < 8; ++g) {
        const v16f& od = w.o[kGive + (g >> 2)];
        const v4f x = {od[4 * (g & 3)], od[4 * (g & 3) + 1], od[4 * (g & 3) + 2], od[4 * (g & 3) + 3]};
        lds_write16(base + (uint32_t)(GB ? g : 8 + g) * 1024u, __builtin_bit_cast(v4i, x));
    }
    *(LDS_AS v2i*)(uintptr_t)(base + 16u * 1024u + (GB ? 8u : 0u)) = (v2i){__builtin_bit_cast(int, l_own), (int)w.bw};
    block_barrier();
    const v2i so = *(const LDS_AS v2i*)(uintptr_t)(base + 16u * 1024u + (GB ? 0u : 8u));
    const float l_a = GB ? __builtin_bit_cast(float, so[0]) : l_own;
    const float l_b = GB ? l_own : __builtin_bit_cast(float, so[0]);
    const uint32_t bw_a = GB ? (uint32_t)so[1] : w.bw;
    const uint32_t bw_b = GB ? w.bw : (uint32_t)so[1];
    const float b_a = bias_of(bw_a), b_b = bias_of(bw_b);
    const bool keep_a = b_a <= b_b;
    const float sc = __builtin_amdgcn_exp2f(512.0f * (keep_a ? b_a - b_b : b_b - b_a));
    const float sa = keep_a ? 1.0f : sc, sb = keep_a ? sc : 1.0f;
#pragma unroll
    for (int g = 0; g < 8; ++g) {
        const v4f ot = __builtin_bit_cast(v4f, lds_read16(base + (uint32_t)(GB ? 8 + g : g) * 1024u));
        v16f& od = w.o[kKeep + (g >> 2)];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float oa = GB ? ot[e] : od[4 * (g & 3) + e];
            const float ob = GB ? od[4 * (g & 3) + e] : ot[e];
            od[4 * (g & 3) + e] = __builtin_fmaf(ob, sb, oa * sa);
        }
    }
    const float l = __builtin_fmaf(l_b, sb, l_a * sa);
    w.lacc[0] = l;
    w.lacc[1] = l;
    w.bw = keep_a ? bw_a : bw_b;
}

// Two 4-wave groups one phase apart (waves 0-3: A, 4-7: B; the hardware places waves w and w + 4 on one SIMD).
// Per tile each wave runs a VALU phase V(t) (rebase, P, the operand prefetch of QK(t+1)) and an MFMA phase M(t)
// (QK(t+1), then PV(t)); one wave of every SIMD pair converts while the other multiplies, and s_setprio hands the
// MFMA-phase wave the issue priority. The staging schedule is in the loop below.
//
// HV (blocks with at most 128 query rows): both groups take rows 0..127 (wave w and w + 4 the same 32) and split every
// tile's keys instead, A keys 0..63 and B keys 64..127 (two of the four 32-key accumulators, half the MFMAs); the
// schedule, the ring and the copies are unchanged. After the loop B hands its softmax state to A through LDS and A
// merges the two (merge_halves).
template <bool LUT, bool SPLIT, bool GB, bool VS, bool HV, bool SC>
__device__ __forceinline__ void attend_pingpong_group(const Prm& p, uint32_t lds, uint32_t qtile, uint32_t head, uint32_t bidx,
                                                      uint32_t split, uint32_t key_lo, uint32_t key_hi) {
    constexpr int NT = 512;
    constexpr int NA = HV ? 2 : 4;              // 32-key accumulators per tile and wave
    constexpr int KB0 = HV && GB ? 2 : 0;       // the first of them
    const Recipe rc = recipe(LUT);
    // rows per block: 256, or 128 for the full-sequence split-tile kernel (the KV split's split-tile blocks keep the
    // 256-row grid and use their first 128 rows)
    constexpr uint32_t RB = HV && !SPLIT ? 128u : 256u;
    const uint32_t tblk = ((bidx * p.splits + split) * p.H + head) * ((p.S + RB - 1u) / RB) + qtile;   // trace slot
    (void)tblk;
    FMHA_MARK(p, tblk, 0);
#ifdef FMHA_TRACE
    if (p.trace && (threadIdx.x & 63u) == 0u) p.trace[((size_t)tblk * 8u + (threadIdx.x >> 6)) * 8u + 7u] = p.t_entry;
#endif
    Wave<NT> w;
    w.init(p, lds, qtile, head, bidx, key_hi, HV ? wave_id() & 3u : wave_id(), RB);
    FMHA_MARK(p, tblk, 1);
    const uint32_t kvh = head / p.gqa;
    const bool causal = (p.flags & 1u) != 0;
    uint32_t key_end = key_hi;   // the block's last useful key + 1
    if (causal) key_end = (uint32_t)max(0, min((int)key_hi, (int)(qtile * RB + RB - 1) + (int)p.SK - (int)p.S + 1));
    const uint32_t ntiles = key_end > key_lo ? (key_end - key_lo + kTile - 1) / kTile : 0;

    Stager<NT> st;
    st.init(p.k + (size_t)bidx * p.k_b + kvh * kD, p.v + (size_t)bidx * p.v_b + kvh * kD, p.ks + (size_t)bidx * p.ks_b + kvh * 4u,
            p.k_seq, p.SK, lds);
    if (VS) st.init_vs(p.vs32 + (size_t)bidx * p.vs_b + kvh * kD, p.vs_row);
    auto slot_of = [](uint32_t t) { return t & 3u; };
    auto key_of = [&](uint32_t t) { return key_lo + t * kTile; };

    v16f s[NA];
    FMHA_LDECL;
    if (ntiles > 0) {
        // One barrier per tile. Group A (waves 0-3) runs  V(t) | barrier | M(t),  group B (waves 4-7)  V(t) M(t) |
        // barrier, so the interval I(t) between barriers t-1 and t holds A: M(t-1), V(t) and B: V(t), M(t): each SIMD
        // holds one wave of each group, and one converts while the other multiplies without a barrier in between.
        // Reads of tile u: K u in I(u-1) (both prefetches, B's QK) and I(u) (A's QK); V u in I(u) (B) and I(u+1) (A);
        // the K-scale words of u in I(u-1) only (the prefetch keeps them in registers).
        // K/V tiles go HBM -> LDS by direct copies: V(t) issues K tile t+3 and V tile t+2 (slot u & 3), and the barrier
        // that ends I(t+1) waits for them (each wave's vmcnt wait there leaves only the copies of its own V(t+1) in
        // flight, and the barrier makes every wave's copies visible): the first reads, in I(t+2), come after it. The
        // slots written in I(t), K (t-1) & 3 and V (t-2) & 3, were last read in I(t-1). The K-scale words go through
        // registers: V(t) loads tile t+3's and stores tile t+2's (slot (t+2) & 3, last read in I(t-3)), published by
        // barrier t. A copy past the range (an empty resource) writes zeros into its slot, which is free as above.
        constexpr int kDmaOps = 2 * Stager<NT>::kN + 1 + (VS ? 1 : 0);   // VMEM operations issued per VALU phase
        // Every prologue load goes out at once (Q and its scales were issued by init): the K-scale words of tiles 0..2,
        // then the copies. One memory round trip to the first barrier (the stores of the words wait for their loads).
        st.init_dma();
        const uint32_t ks0 = st.ks_word(key_of(0), true);
        const uint32_t ks1 = st.ks_word(key_of(1), ntiles > 1);
        st.load_ks(key_of(2), ntiles > 2);                              // stored by V(0)
        // The first barrier needs K 0, V 0 and K 1 (read in I(0)); V 1 and K 2 are first read in I(1), so barrier 0
        // waits for them and they stay out of the first barrier's burst.
        st.dma(key_of(0), true, 0, key_of(0), true, 0);                 // K 0, V 0
        st.dma(key_of(1), ntiles > 1, 1, key_of(1), false, 3);          // K 1 (V slot 3 gets zeros, nothing reads it yet)
        if (VS) st.dma_vs(key_of(0), true, 0);                          // V scales of tile 0
        // The stores of the words wait for their loads. The compiler counts only its own loads (not the copies' inline
        // assembly), so its wait there leaves at most two VMEM operations of any kind in flight: placed before the
        // copies of K 2 and V 1, it does not hold the first barrier for those two (kvsplit kernel alone at cfg5
        // -2.4 %, cfg3 -0.6 %).
        st.store_ks_word(ks0, 0);
        st.store_ks_word(ks1, 1);
        w.commit_q();   // (its wait for the Q scale word likewise comes before the copies of K 2 and V 1)
        st.dma(key_of(2), ntiles > 2, 2, key_of(1), ntiles > 1, 1);     // K 2, V 1
        if (VS) st.dma_vs(key_of(1), ntiles > 1, 1);                    // V scales of tile 1
        // everything but the copies of K 2 and V 1 (which barrier 0 waits for)
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * Stager<NT>::kN + (VS ? 1 : 0)) : "memory");
        FMHA_MARK(p, tblk, 2);
        block_barrier();
        FMHA_MARK(p, tblk, 3);
        w.template qk_all<KB0>(0, s);
        float mrow = row_max(s);   // unmasked row max of the tile the next VALU phase decides on
        {
            typename Wave<NT>::Ring ring;
            typename Wave<NT>::QkPre pre;
            // V(t)'s copies: K tile t+3 and V tile t+2 (and the per-32-key V scales), the K-scale words of tile t+3
            auto copies = [&](uint32_t t) {
                st.dma(key_of(t + 3), t + 3 < ntiles, slot_of(t + 3), key_of(t + 2), t + 2 < ntiles, slot_of(t + 2));
                if (VS) st.dma_vs(key_of(t + 2), t + 2 < ntiles, slot_of(t + 2));
                st.load_ks(key_of(t + 3), t + 3 < ntiles);
            };
            auto v_phase = [&](uint32_t t, uint32_t (&pw)[NA][4], bool last) {
                FMHA_SETPRIO(0);
                st.store_ks(slot_of(t + 2));
                if (SC) w.scale_s(s, mrow);   // the in-kernel softmax scale (an instantiation of its own)
                if (w.needs_mask(key_of(t))) {
                    w.template apply_mask<KB0>(s, key_of(t));
                    mrow = row_max(s);
                }
                rebase<LUT>(rc, mrow, s, w.o, w.lacc, w.bias, w.bw, w.qrm);
                // the tile copies go out between the rebase decision and the conversion: A/B on one box, -0.3 % at
                // cfg2 and -0.4 % at cfg3 against issuing them first (after the conversion: the same; after the
                // prefetch: +0.4 %)
                copies(t);
#pragma unroll
                for (int t4 = 0; t4 < NA; ++t4) convert_p<LUT>(rc, s[t4], pw[t4]);
                if (!last) {
                    s[NA - 1] = splat16(w.bias);
                    w.template qk_prefetch<NA, KB0>(slot_of(t + 1), ring, pre);
                }

                FMHA_LMARK(p, tblk, t, 0);
                // A: the copies of the previous VALU phase have landed; this phase's and the prefetched reads stay in flight
                if (!GB) block_barrier_keep_dma<2 * Wave<NT>::DEPTH, kDmaOps>();
                if (GB) asm volatile("" ::: "memory");
                FMHA_LMARK(p, tblk, t, 1);
                FMHA_SETPRIO(1);
            };
            uint32_t t = 0;
            for (; t + 1 < ntiles; ++t) {
                uint32_t pw[NA][4];
                v_phase(t, pw, false);
                mrow = w.template m_phase_qf<true, VS, KB0>(slot_of(t), pw, slot_of(t + 1), s, ring, pre);
                FMHA_LMARK(p, tblk, t, 2);
                if (GB) block_barrier_keep_dma<0, kDmaOps>();
                else asm volatile("" ::: "memory");   // A: the compiler-only fence where B has its barrier
                FMHA_LMARK(p, tblk, t, 3);
            }
            {
                // the last tile: PV only
                uint32_t pw[NA][4];
                v_phase(t, pw, true);
                (void)w.template m_phase_qf<false, VS, KB0>(slot_of(t), pw, slot_of(t), s, ring, pre);
                if (GB) block_barrier();
            }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // no copy into LDS outlives the loop
        FMHA_SETPRIO(0);
    }
    FMHA_MARK(p, tblk, 4);
    FMHA_LFLUSH(p, tblk);
    if (!HV) {
        epilogue<SPLIT, NT, GB>(p, w, head, bidx, split, rc, true);
    } else {
        // HV: each group finishes half of every row's dims (A 0..63, B 64..127); the merge's barriers retired the ring
        merge_halves<GB>(w, lds);
        FMHA_MARK(p, tblk, 6);
        epilogue<SPLIT, NT, false, GB ? 2 : 1>(p, w, head, bidx, split, rc, false);
    }
    FMHA_MARK(p, tblk, 5);
}

// The whole routine is instantiated per group (the groups place their barrier differently; one body with a
// group-dependent branch, or two loop copies sharing a prologue, made the register allocation spill).
template <bool LUT, bool SPLIT, bool VS, bool HV, bool SC>
__device__ __forceinline__ void attend_pingpong(const Prm& p, uint32_t lds, uint32_t qtile, uint32_t head, uint32_t bidx, uint32_t split,
                                uint32_t key_lo, uint32_t key_hi) {
    if (wave_id() >= 4u) attend_pingpong_group<LUT, SPLIT, true, VS, HV, SC>(p, lds, qtile, head, bidx, split, key_lo, key_hi);
    else attend_pingpong_group<LUT, SPLIT, false, VS, HV, SC>(p, lds, qtile, head, bidx, split, key_lo, key_hi);
}

// One 4-wave block of 128 rows with one wave per SIMD (_t128 under its own 256-thread contract). Nothing else runs on
// the wave's SIMD, so each wave overlaps its own VALU work with its own MFMAs (m_phase_cv): iteration t runs QK(t+1)
// with the conversion of P(t), then PV(t) with the row max of S(t+1), then (behind the tile's barrier) the rebase
// decision of S(t+1). S(t) and S(t+1) live in two register sets that swap roles every iteration (the loop body is
// instantiated twice). Every copy of a tile is direct HBM -> LDS: K and V into a 4-slot ring, the K-scale words
// (unshifted, kscale_raw) and the V scales into their 4-slot rings. Iteration t issues tile t+3's copies, one behind
// each of its first MFMAs, into slot (t+3) & 3; it reads K(t+1) and V(t), and the slots it writes, K (t-1) & 3 (last
// read in iteration t-2) and V (t-1) & 3 (iteration t-1), are free behind barrier t-1. Each barrier waits for the
// copies of the iteration before: tile t+2 has landed before barrier t, an iteration ahead of its first read.
template <bool LUT, bool VS, bool SC>
__device__ __forceinline__ void attend_single_wave(const Prm& p, uint32_t lds, uint32_t qtile, uint32_t head, uint32_t bidx) {
    constexpr int NT = 256;
    const Recipe rc = recipe(LUT);
    const uint32_t tblk = (bidx * p.H + head) * ((p.S + 127u) / 128u) + qtile;
    (void)tblk;
    FMHA_MARK(p, tblk, 0);
#ifdef FMHA_TRACE
    if (p.trace && (threadIdx.x & 63u) == 0u) p.trace[((size_t)tblk * 8u + (threadIdx.x >> 6)) * 8u + 7u] = p.t_entry;
#endif
    Wave<NT> w;
    w.init(p, lds, qtile, head, bidx, p.SK, wave_id());
    FMHA_MARK(p, tblk, 1);
    const uint32_t kvh = head / p.gqa;
    const bool causal = (p.flags & 1u) != 0;
    uint32_t key_end = p.SK;
    if (causal) key_end = (uint32_t)max(0, min((int)p.SK, (int)(qtile * 128u + 127u) + (int)p.SK - (int)p.S + 1));
    const uint32_t ntiles = (key_end + kTile - 1) / kTile;
    Stager<NT> st;
    st.init(p.k + (size_t)bidx * p.k_b + kvh * kD, p.v + (size_t)bidx * p.v_b + kvh * kD, p.ks + (size_t)bidx * p.ks_b + kvh * 4u,
            p.k_seq, p.SK, lds);
    if (VS) st.init_vs(p.vs32 + (size_t)bidx * p.vs_b + kvh * kD, p.vs_row);
    auto key_of = [](uint32_t t) { return t * kTile; };
    auto slot_of = [](uint32_t t) { return t & 3u; };
    FMHA_LDECL;
    if (ntiles > 0) {
        st.init_dma();
        // every copy of a tile: K, V, the K-scale words and (extension) the V scales; all three prologue tiles at once
        auto copy_tile = [&](uint32_t u) {
            st.dma(key_of(u), u < ntiles, slot_of(u), key_of(u), u < ntiles, slot_of(u));
            st.dma_ks(key_of(u), u < ntiles, slot_of(u));
            if (VS) st.dma_vs(key_of(u), u < ntiles, slot_of(u));
        };
        copy_tile(0);
        copy_tile(1);
        // the compiler's wait for the Q scale word (it does not count the copies' inline assembly) comes before tile
        // 2's copies, so that it does not hold the first barrier for them (cfg1 -1.5 %)
        w.commit_q();
        copy_tile(2);
        // VMEM operations per tile: the K and V copies, the K-scale copy and (extension) the V-scale copy
        constexpr int kOps = 2 * Stager<NT>::kN + 1 + (VS ? 1 : 0);
        FMHA_MARK(p, tblk, 2);
        block_barrier_keep_dma<0, kOps>();   // tiles 0 and 1 have landed; tile 2's copies stay in flight
        FMHA_MARK(p, tblk, 3);
        v16f sa[4], sb[4];
        {
            w.template qk_all<0, 4, true>(0, sa);
            float m0 = row_max(sa);
            if (SC) w.scale_s(sa, m0);
            if (w.needs_mask(key_of(0))) {
                w.apply_mask(sa, key_of(0));
                m0 = row_max(sa);
            }
            rebase<LUT>(rc, m0, sa, w.o, w.lacc, w.bias, w.bw, w.qrm);
        }
        uint32_t t = 0;
        // iteration t: S(t) in sc (rebased), S(t+1) into sn
        auto step = [&](v16f (&sc)[4], v16f (&sn)[4]) {
            FMHA_LMARK(p, tblk, t, 0);
            uint32_t pw[4][4];
            // the copies of tile t+3, one instruction behind each of the phase's first MFMAs
            const uint32_t u = t + 3;
            auto copies = [&](int i) {
                if (i < 2 * Stager<NT>::kN) st.dma_part(i, key_of(u), u < ntiles, slot_of(u));
                else if (i == 2 * Stager<NT>::kN) st.dma_ks(key_of(u), u < ntiles, slot_of(u));
                else if (VS && i == 2 * Stager<NT>::kN + 1) st.dma_vs(key_of(u), u < ntiles, slot_of(u));
            };
            float m = w.template m_phase_cv<LUT, VS, true>(rc, slot_of(t), slot_of(t + 1), sc, sn, pw, copies);
            if (SC) w.scale_s(sn, m);
            if (w.needs_mask(key_of(t + 1))) {
                w.apply_mask(sn, key_of(t + 1));
                m = row_max(sn);
            }
            FMHA_LMARK(p, tblk, t, 1);
            block_barrier_keep_dma<0, kOps>();   // tile t+2 has landed (this iteration's operations stay in flight)
            FMHA_LMARK(p, tblk, t, 2);
            rebase<LUT>(rc, m, sn, w.o, w.lacc, w.bias, w.bw, w.qrm);
            FMHA_LMARK(p, tblk, t, 3);
            ++t;
        };
        auto last = [&](v16f (&sc)[4]) {
            uint32_t pw[4][4];
            (void)w.template m_phase_cv<LUT, VS, false>(rc, slot_of(t), slot_of(t), sc, sc, pw, [](int) {});
        };
        // two iterations per trip, so the sets swap without copies (one copy when the last tile's S is in sb: with a
        // second instantiation of the last tile the register allocation spilled)
        while (t + 1 < ntiles) {
            step(sa, sb);
            if (t + 1 >= ntiles) {
#pragma unroll
                for (int a = 0; a < 4; ++a) sa[a] = sb[a];
                break;
            }
            step(sb, sa);
        }
        last(sa);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // no copy into LDS outlives the loop
    }
    FMHA_MARK(p, tblk, 4);
    FMHA_LFLUSH(p, tblk);
    epilogue<false>(p, w, head, bidx, 0, rc, true);
    FMHA_MARK(p, tblk, 5);
}

// Workgroup -> (q tile, head, z): consecutive tiles of one (batch, head) land on one XCD, so each XCD's L2 holds the K/V
// its blocks share. The hardware deals workgroups round-robin over the 8 XCDs in linear order x + gx (y + gy z); when
// n = gx gy is a multiple of 8 that XCD is (x + gx y) mod 8 in every z slice, and L -> (L mod 8) (n / 8) + L / 8
// gives XCD k the slice's logical blocks [k n / 8, (k + 1) n / 8). The grid extents come from the kernel arguments
// (gx = ceil(S / rows), gy = H): reading them from the dispatch packet, which sits in the host-memory queue, cost every
// wave a round trip over PCIe at start-up (microseconds, growing with the wave count).
// pair: the causal q-tile pairing (FMHA_FLAG_CAUSAL_PAIR): the grid's x extent is ceil(T / 2) for T query tiles.
__device__ inline void block_coords(uint32_t S, uint32_t H, uint32_t rows, uint32_t& qt, uint32_t& head, uint32_t& z, bool pair = false) {
    const uint32_t nt = (S + rows - 1u) / rows;
    const uint32_t gx = pair ? (nt + 1u) / 2u : nt;
    const uint32_t n = gx * H;
    uint32_t L = blockIdx.x + gx * blockIdx.y;
    if ((n & 7u) == 0u) L = (L & 7u) * (n >> 3) + (L >> 3);
    qt = __builtin_amdgcn_readfirstlane(L % gx);
    head = __builtin_amdgcn_readfirstlane(L / gx);
    z = blockIdx.z;
}

// Inlined into its kernel, like everything that reads the kernel arguments: in a called (outlined) function the
// kernarg segment pointer is not an ABI input and compiles to null. build.py rejects a code object with a call.
// SC: the `_scaled` kernel of the pair (the softmax scale at 0x050 applied in the kernel).
template <int NT, bool SC>
__device__ __forceinline__ void full_kernel(uint32_t lds) {
#ifdef FMHA_TRACE
    const uint64_t t_entry = __builtin_amdgcn_s_memrealtime();
    Prm p = prm_from_kernarg<SC>();
    p.t_entry = t_entry;
#else
    const Prm p = prm_from_kernarg<SC>();
#endif
    const bool lut = (p.SK + 127u) / 128u < 4u;   // state.rs:75-77
    if constexpr (NT == 512) {
        uint32_t qt, head, z;
        block_coords(p.S, p.H, 256u, qt, head, z);
        if (p.vs32) {
            if (lut) attend_pingpong<true, false, true, false, SC>(p, lds, qt, head, z, 0, 0, p.SK);
            else attend_pingpong<false, false, true, false, SC>(p, lds, qt, head, z, 0, 0, p.SK);
        } else {
            if (lut) attend_pingpong<true, false, false, false, SC>(p, lds, qt, head, z, 0, 0, p.SK);
            else attend_pingpong<false, false, false, false, SC>(p, lds, qt, head, z, 0, 0, p.SK);
        }
    } else {
        // the causal q-tile pairing (FMHA_FLAG_CAUSAL_PAIR, 128-row grids only: the 256-row kernel's registers have no
        // room for the pass loop, and validate refuses the flag for it; grid.rs:94-111): block x runs q tiles x and
        // T - 1 - x (the second only when it is past x), so every block does the same work; a barrier between passes
        uint32_t x, head, z;
        const bool pair = (p.flags & FMHA_FLAG_CAUSAL_PAIR) != 0u;
        block_coords(p.S, p.H, 128u, x, head, z, pair);
        const uint32_t nt = (p.S + 127u) / 128u;
        const uint32_t npass = pair && nt - 1u - x > x ? 2u : 1u;
        for (uint32_t pass = 0; pass < npass; ++pass) {
            const uint32_t qt = pass == 0u ? x : nt - 1u - x;
            if (pass > 0u) block_barrier();
            if (p.vs32) {
                if (lut) attend_single_wave<true, true, SC>(p, lds, qt, head, z);
                else attend_single_wave<false, true, SC>(p, lds, qt, head, z);
            } else {
                if (lut) attend_single_wave<true, false, SC>(p, lds, qt, head, z);
                else attend_single_wave<false, false, SC>(p, lds, qt, head, z);
            }
        }
    }
}

// The KV-split kernel body (SC as in full_kernel).
template <bool SC>
__device__ __forceinline__ void kvsplit_kernel(uint32_t smem_base) {
#ifdef FMHA_TRACE
    const uint64_t t_entry = __builtin_amdgcn_s_memrealtime();
    Prm p = prm_from_kernarg<SC, true>();
    p.t_entry = t_entry;
#else
    Prm p = prm_from_kernarg<SC, true>();
#endif
    p.flags = 0;   // 0x280 holds the split count in this layout
    p.lse_out = nullptr;
    p.ohat = (uint8_t*)ka<uint64_t>(offsetof(fmha_mxfp8_kvsplit_args, ptr_ohat));
    p.lse = (float*)ka<uint64_t>(offsetof(fmha_mxfp8_kvsplit_args, ptr_lse));
    const uint32_t split_field = ka<uint32_t>(offsetof(fmha_mxfp8_kvsplit_args, kvs_splits));
    p.splits = split_field & 0xffffu;
    p.f32_partials = (split_field & FMHA_KVS_F32_PARTIALS) ? 1u : 0u;
    p.vs32 = (split_field & FMHA_KVS_V_SEQ32) ? (const uint8_t*)p.vd : nullptr;   // 0x280 is not `flags` here
    p.rows_total = ka<uint32_t>(offsetof(fmha_mxfp8_kvsplit_args, kvs_rows_total));
    uint32_t qt, head, z;
    const uint32_t gz = p.rows_total / (p.S * p.H) * p.splits;   // B x splits (rows_total = B S H: validate's rule)
    if ((p.S + 255u) / 256u == 1u && (gz & 7u) == 0u) {
        // One query tile per (batch, head, split): no two blocks share K/V rows, so the XCD placement serves the LSE
        // words instead. Block L of the (H, gz) grid goes to XCD L mod 8; L -> z = (L mod 8) + 8 ((L / 8) / H),
        // head = (L / 8) mod H puts the H heads of one split on one XCD, and the H consecutive LSE words of a row
        // (row index (b S + s) H + h) meet in one L2, which writes them back as whole lines.
        const uint32_t L = blockIdx.y + p.H * blockIdx.z, j = L >> 3;
        qt = 0;
        head = __builtin_amdgcn_readfirstlane(j % p.H);
        z = __builtin_amdgcn_readfirstlane((L & 7u) + 8u * (j / p.H));
    } else {
        block_coords(p.S, p.H, 256u, qt, head, z);
    }
    // components.rs:20-30 / 58-74: z = batch * splits + split; split s owns tiles [s tps, min(ntiles, (s+1) tps))
    const uint32_t bidx = z / p.splits, split = z % p.splits;
    const uint32_t ntiles = (p.SK + 127u) / 128u;
    const uint32_t tps = (ntiles + p.splits - 1u) / p.splits;
    const uint32_t tile_lo = split * tps;
    const uint32_t tile_hi = min(ntiles, tile_lo + tps);
    const uint32_t key_lo = tile_lo * 128u, key_hi = min(tile_hi * 128u, p.SK);
    const bool lut = ntiles < 4u;
    // a block with at most 128 query rows (decode-like S; the ragged last block) splits each tile's keys between the
    // two wave groups instead of leaving the second group on padding rows (the LUT recipe, SK < 512, keeps the plain
    // order)
    const bool hv = !lut && p.S - qt * 256u <= 128u;
    if (p.vs32) {
        if (lut) attend_pingpong<true, true, true, false, SC>(p, smem_base, qt, head, bidx, split, key_lo, key_hi);
        else if (hv) attend_pingpong<false, true, true, true, SC>(p, smem_base, qt, head, bidx, split, key_lo, key_hi);
        else attend_pingpong<false, true, true, false, SC>(p, smem_base, qt, head, bidx, split, key_lo, key_hi);
    } else {
        if (lut) attend_pingpong<true, true, false, false, SC>(p, smem_base, qt, head, bidx, split, key_lo, key_hi);
        else if (hv) attend_pingpong<false, true, false, true, SC>(p, smem_base, qt, head, bidx, split, key_lo, key_hi);
        else attend_pingpong<false, true, false, false, SC>(p, smem_base, qt, head, bidx, split, key_lo, key_hi);
    }
}

// The full-sequence split-tile kernel (extension): the t128 grid (128 query rows per block) with 512 threads; both wave
// groups take the block's rows and split each tile's keys (HV), so one group converts while the other multiplies,
// which one wave per SIMD cannot do. The host launches it for t128's shapes with the non-LUT recipe; the LUT case is
// served too (the merge is exact either way), for direct launches.
template <bool SC>
__device__ __forceinline__ void t128_split_tiles_kernel(uint32_t lds) {
#ifdef FMHA_TRACE
    const uint64_t t_entry = __builtin_amdgcn_s_memrealtime();
    Prm p = prm_from_kernarg<SC>();
    p.t_entry = t_entry;
#else
    const Prm p = prm_from_kernarg<SC>();
#endif
    uint32_t x, head, z;
    const bool pair = (p.flags & FMHA_FLAG_CAUSAL_PAIR) != 0u;
    block_coords(p.S, p.H, 128u, x, head, z, pair);
    const bool lut = (p.SK + 127u) / 128u < 4u;   // state.rs:75-77
    const uint32_t nt = (p.S + 127u) / 128u;
    const uint32_t npass = pair && nt - 1u - x > x ? 2u : 1u;   // the causal q-tile pairing, as in full_kernel
    for (uint32_t pass = 0; pass < npass; ++pass) {
        const uint32_t qt = pass == 0u ? x : nt - 1u - x;
        if (pass > 0u) block_barrier();
        if (p.vs32) {
            if (lut) attend_pingpong<true, false, true, true, SC>(p, lds, qt, head, z, 0, 0, p.SK);
            else attend_pingpong<false, false, true, true, SC>(p, lds, qt, head, z, 0, 0, p.SK);
        } else {
            if (lut) attend_pingpong<true, false, false, true, SC>(p, lds, qt, head, z, 0, 0, p.SK);
            else attend_pingpong<false, false, false, true, SC>(p, lds, qt, head, z, 0, 0, p.SK);
        }
    }
}

}  // namespace

#define FMHA_LDS_BASE(name)                                                 \
    __shared__ __attribute__((aligned(1024))) uint8_t name[kLdsBytes]; \
    const uint32_t name##_base = (uint32_t)(uintptr_t)(LDS_AS uint8_t*)name

extern "C" __global__ void __launch_bounds__(512, 1) fmha_fwd_hd128_mxfp8_v3_vs128(fmha_mxfp8_args a) {
    FMHA_LDS_BASE(smem);
    (void)a;   // read through kernarg()
    full_kernel<512, false>(smem_base);
}

extern "C" __global__ void __launch_bounds__(256, 1) fmha_fwd_hd128_mxfp8_v3_t128(fmha_mxfp8_args a) {
    FMHA_LDS_BASE(smem);
    (void)a;
    full_kernel<256, false>(smem_base);
}

extern "C" __global__ void __launch_bounds__(512, 1) fmha_fwd_hd128_mxfp8_v3_kvsplit(fmha_mxfp8_kvsplit_args ka_) {
    FMHA_LDS_BASE(smem);
    (void)ka_;   // read through ka<>(); bytes 0x000..0x26F are the base layout
    kvsplit_kernel<false>(smem_base);
}

// Extension kernels (no counterpart in the reference): the same ABIs, the softmax scale at 0x050 applied in the kernel.
// The host launches them when FMHA_FLAG_SCALE (0x280 of the full-sequence layout) or FMHA_KVS_SCALE (the split
// field) is set; the reference-named kernels ignore 0x050, as the reference's do.
extern "C" __global__ void __launch_bounds__(512, 1) fmha_fwd_hd128_mxfp8_v3_vs128_scaled(fmha_mxfp8_args a) {
    FMHA_LDS_BASE(smem);
    (void)a;
    full_kernel<512, true>(smem_base);
}

extern "C" __global__ void __launch_bounds__(256, 1) fmha_fwd_hd128_mxfp8_v3_t128_scaled(fmha_mxfp8_args a) {
    FMHA_LDS_BASE(smem);
    (void)a;
    full_kernel<256, true>(smem_base);
}

extern "C" __global__ void __launch_bounds__(512, 1) fmha_fwd_hd128_mxfp8_v3_kvsplit_scaled(fmha_mxfp8_kvsplit_args ka_) {
    FMHA_LDS_BASE(smem);
    (void)ka_;
    kvsplit_kernel<true>(smem_base);
}

// Extension kernels (no counterpart in the reference): t128's grid and kernarg layout, 512 threads, split tiles.
extern "C" __global__ void __launch_bounds__(512, 1) fmha_fwd_hd128_mxfp8_v3_t128_split_tiles(fmha_mxfp8_args a) {
    FMHA_LDS_BASE(smem);
    (void)a;
    t128_split_tiles_kernel<false>(smem_base);
}

extern "C" __global__ void __launch_bounds__(512, 1) fmha_fwd_hd128_mxfp8_v3_t128_split_tiles_scaled(fmha_mxfp8_args a) {
    FMHA_LDS_BASE(smem);
    (void)a;
    t128_split_tiles_kernel<true>(smem_base);
}

// epilogue.rs:89-167 / io.rs:164-185: thread t -> 8 consecutive outputs of row t >> 4 (tail threads redo the last group)
// The combines take the 36-byte layout (fmha_mxfp8_combine_args: three pointers, then rows_total, d and the split
// field at 0x18, 0x1C, 0x20) as scalar parameters, which lay out the same bytes: as scalars the nine dwords are preloaded
// into SGPRs by the hardware at wave launch (the build's -amdgpu-kernarg-preload-count), so the kernel starts on its loads
// without a memory round trip for its arguments. (An aggregate parameter is not preloaded.)
#define FMHA_COMBINE_PARAMS \
    const uint8_t* ohat, const float* lse, uint8_t* out, uint32_t rows, uint32_t d, uint32_t split_field
static_assert(offsetof(fmha_mxfp8_combine_args, ptr_ohat) == 0x00 && offsetof(fmha_mxfp8_combine_args, ptr_lse) == 0x08 &&
                  offsetof(fmha_mxfp8_combine_args, ptr_out) == 0x10 && offsetof(fmha_mxfp8_combine_args, rows_total) == 0x18 &&
                  offsetof(fmha_mxfp8_combine_args, d) == 0x1C && offsetof(fmha_mxfp8_combine_args, splits) == 0x20 &&
                  sizeof(fmha_mxfp8_combine_args) == 36,
              "the combine kernels' scalar parameters follow the packed layout");

extern "C" __global__ void __launch_bounds__(256) fmha_fwd_hd128_mxfp8_v3_kvsplit_combine8h(FMHA_COMBINE_PARAMS) {
    (void)d;
    const uint32_t groups = rows << 4;
    uint32_t t = blockIdx.x * 256u + threadIdx.x;
    t = t < groups ? t : groups - 1u;
    const uint32_t splits = split_field & 0xffffu;
    MergeState st;
    merge_init(st);
    if (split_field & FMHA_KVS_F32_PARTIALS) merge_splits<true>(lse, ohat, rows, 0u, splits, t, st);
    else merge_splits<false>(lse, ohat, rows, 0u, splits, t, st);
    store16_system(out + (size_t)t * 16u, merge_finish(st));
}

// Extension (no counterpart in the reference): the same merge for many splits, with the splits spread over the block's
// 4 waves. Lane l of every wave takes group 64 blockIdx.x + l (outputs 8 (g & 15) .. +7 of row g >> 4, tail lanes redo
// the last group); wave p merges the p-th quarter of the splits (ceil(splits / 4) each, in order), and wave 0 merges
// the quarters in order through LDS. With the reference kernel's layout one thread walks every split of its group in
// turn: at 32 splits that is 4 dependent rounds of loads on 64 groups per block (13.7 us at 1024 rows on MI355X).
extern "C" __global__ void __launch_bounds__(256) fmha_fwd_hd128_mxfp8_v3_kvsplit_combine_wide(FMHA_COMBINE_PARAMS) {
    (void)d;
    __shared__ float part[3][10][64];
    const uint32_t splits = split_field & 0xffffu;
    const uint32_t groups = rows << 4;
    const uint32_t lane = threadIdx.x & 63u, p = threadIdx.x >> 6;
    uint32_t t = blockIdx.x * 64u + lane;
    t = t < groups ? t : groups - 1u;
    const uint32_t per = (splits + 3u) >> 2;
    const uint32_t lo = min(p * per, splits), hi = min(lo + per, splits);
    MergeState st;
    merge_init(st);
    if (lo < hi) {
        if (split_field & FMHA_KVS_F32_PARTIALS) merge_splits<true>(lse, ohat, rows, lo, hi, t, st);
        else merge_splits<false>(lse, ohat, rows, lo, hi, t, st);
    }
    if (p != 0u) {
        part[p - 1][0][lane] = st.m;
        part[p - 1][1][lane] = st.den;
#pragma unroll
        for (int i = 0; i < 8; ++i) part[p - 1][2 + i][lane] = st.acc[i];
    }
    __syncthreads();
    if (p != 0u) return;
#pragma unroll
    for (int q = 0; q < 3; ++q) {
        // a quarter past the split count (splits < 4) holds no split: skipped, so the result is the in-order merge
        if ((uint32_t)(q + 1) * per >= splits) break;
        MergeState o;
        o.m = part[q][0][lane];
        o.den = part[q][1][lane];
#pragma unroll
        for (int i = 0; i < 8; ++i) o.acc[i] = part[q][2 + i][lane];
        merge_states(st, o);
    }
    store16_system(out + (size_t)t * 16u, merge_finish(st));
}
