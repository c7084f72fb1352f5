/*
 * fmha_mxfp8.h - C ABI of the MI355X (gfx950) MXFP8 FMHA forward, head dim 128.
 *
 * Drop-in boundary for the reference's `fmha_fwd_hd128_mxfp8_auto` path
 * (demonsan/AMDGPU_RustDSL). Everything here is plain C: pointers, sizes and
 * 32-bit integers; no HIP, torch or C++ types appear in a signature.
 *
 * The four kernels live in one code object that this library embeds and loads
 * with hipModuleLoadData; they keep the reference's symbol names
 *   fmha_fwd_hd128_mxfp8_v3_vs128             (tests/gpu/ref_host.cpp:62)
 *   fmha_fwd_hd128_mxfp8_v3_t128              (tests/gpu/ref_host.cpp:67)
 *   fmha_fwd_hd128_mxfp8_v3_kvsplit           (tests/gpu/ref_host.cpp:71)
 *   fmha_fwd_hd128_mxfp8_v3_kvsplit_combine8h (tests/gpu/ref_host.cpp:75)
 * and read a by-value kernarg segment with the byte layout of the structs
 * below, so a launcher written against the reference's generated headers
 * (tests/gpu/generated/, one _abi.h per kernel) launches them unchanged.
 *
 * Numerics (all four kernels): softmax base 2 of dequant(Q).dequant(K)^T with
 * the caller folding log2(e)/sqrt(128) into Q before quantisation
 * (tests/gpu/ref_host.cpp:209-211); kernarg 0x050 (softmax scale) is ignored,
 * as in the reference MX kernels (crates/amdgpu-stage/src/attention/block3.rs:160).
 */
#ifndef FMHA_MXFP8_H
#define FMHA_MXFP8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------- */
/* Kernarg segments                                                          */
/* ------------------------------------------------------------------------- */

#pragma pack(push, 1)
/* The 656-byte kernarg of _vs128 / _t128.
 * Replaces amdc_hostgen::fmha_fwd_hd128_mxfp8_v3_{vs128,t128}::Args
 * (tests/gpu/generated/fmha_fwd_hd128_mxfp8_v3_vs128_abi.h:10-126). */
typedef struct fmha_mxfp8_args {
    void* ptr_o;              /* 0x000 bf16 [B,S,H,128] */
    uint8_t _pad0[8];
    void* ptr_q;              /* 0x010 e4m3 [B,S,H,128] */
    uint8_t _pad1[8];
    void* ptr_k;              /* 0x020 e4m3 [B,SK,HK,128] */
    uint8_t _pad2[8];
    void* ptr_v;              /* 0x030 e4m3 [B,SK,HK,128] */
    uint8_t _pad3[8];
    void* ptr_lse;            /* 0x040 optional f32 [B,H,S] natural-log LSE (extension; NULL = not written) */
    uint8_t _pad3b[8];
    uint32_t softmax_scale;   /* 0x050 f32 bits, ignored (scale folded into Q) */
    uint8_t _pad3c[12];
    uint32_t s_seq_len;       /* 0x060 S */
    uint8_t _pad4[12];
    uint32_t s_Seqs;          /* 0x070 Q row stride = H*128 */
    uint8_t _pad5[28];
    uint32_t s_Hs;            /* 0x090 128 */
    uint8_t _pad6[12];
    uint32_t s_Bs;            /* 0x0A0 S*H*128 */
    uint8_t _pad7[12];
    uint32_t s_gqa;           /* 0x0B0 H/HK, power of two <= 16 */
    uint8_t _pad8[12];
    uint32_t s_k_Seqs;        /* 0x0C0 HK*128 */
    uint8_t _pad9[12];
    uint32_t s_k_Hs;          /* 0x0D0 128 */
    uint8_t _pad10[12];
    uint32_t s_k_Bs;          /* 0x0E0 SK*HK*128 */
    uint8_t _pad11[12];
    uint32_t opt;             /* 0x0F0 ignored (the reference's hand path passes 5) */
    uint8_t _pad11b[28];
    uint32_t s_kv_seq_len;    /* 0x110 SK */
    uint8_t _pad12[44];
    uint32_t s_q_head_num;    /* 0x140 H */
    uint8_t _pad13[12];
    uint32_t s_v_Seqs;        /* 0x150 */
    uint8_t _pad14[12];
    uint32_t s_v_Hs;          /* 0x160 */
    uint8_t _pad15[12];
    uint32_t s_v_Bs;          /* 0x170 */
    uint8_t _pad16[12];
    uint32_t s_o_Seqs;        /* 0x180 H*256 */
    uint8_t _pad17[12];
    uint32_t s_o_Hs;          /* 0x190 256 */
    uint8_t _pad18[12];
    uint32_t s_o_Bs;          /* 0x1A0 S*H*256 */
    uint8_t _pad19[92];
    void* ptr_q_descale;      /* 0x200 E8M0 [B,S,H,4] + zeroed slack */
    uint8_t _pad20[8];
    void* ptr_k_descale;      /* 0x210 E8M0 [B,SK,HK,4] + zeroed slack */
    uint8_t _pad21[8];
    void* ptr_v_descale;      /* 0x220 one f32 in a >= 4096-byte buffer */
    uint8_t _pad22[8];
    uint32_t s_descale_q_Bs;  /* 0x230 S*H*4 */
    uint8_t _pad23[12];
    uint32_t s_descale_q_Hs;  /* 0x240 4 */
    uint8_t _pad24[12];
    uint32_t s_descale_k_Bs;  /* 0x250 SK*HK*4 */
    uint8_t _pad25[12];
    uint32_t s_descale_k_Hs;  /* 0x260 4 */
    uint8_t _pad26[28];
    uint32_t flags;           /* 0x280 extension flags, 0 = reference semantics: FMHA_FLAG_CAUSAL, FMHA_FLAG_V_SEQ32, FMHA_FLAG_SCALE */
    uint8_t abi_tail[12];     /* 0x284 */
} fmha_mxfp8_args;

/* The 648-byte kernarg of _kvsplit: the 656-byte layout up to 0x270, then the
 * split extension. Replaces amdc_hostgen::fmha_fwd_hd128_mxfp8_v3_kvsplit::Args
 * (tests/gpu/generated/fmha_fwd_hd128_mxfp8_v3_kvsplit_abi.h, offsets 0x270-0x284). */
typedef struct fmha_mxfp8_kvsplit_args {
    uint8_t base[0x270];      /* fmha_mxfp8_args bytes 0x000..0x26F */
    void* ptr_ohat;           /* 0x270 fp16 partial rows, 256 B each, split stride rows_total*256 B
                                 (FMHA_KVS_F32_PARTIALS: f32 rows, 512 B each, split stride rows_total*512 B) */
    void* ptr_lse;            /* 0x278 f32 base-2 LSE per partial row */
    uint32_t kvs_splits;      /* 0x280 2, 4 or 8, optionally OR FMHA_KVS_F32_PARTIALS */
    uint32_t kvs_rows_total;  /* 0x284 B*S*H */
} fmha_mxfp8_kvsplit_args;

/* The 36-byte kernarg of _kvsplit_combine8h. Replaces
 * amdc_hostgen::fmha_fwd_hd128_mxfp8_v3_kvsplit_combine8h::Args
 * (tests/gpu/generated/fmha_fwd_hd128_mxfp8_v3_kvsplit_combine8h_abi.h:10-34). */
typedef struct fmha_mxfp8_combine_args {
    void* ptr_ohat;           /* 0x00 */
    void* ptr_lse;            /* 0x08 */
    void* ptr_out;            /* 0x10 bf16 [rows_total,128] */
    uint32_t rows_total;      /* 0x18 */
    uint32_t d;               /* 0x1C 128 */
    uint32_t splits;          /* 0x20 optionally OR FMHA_KVS_F32_PARTIALS */
} fmha_mxfp8_combine_args;
#pragma pack(pop)

/* Extension (no counterpart in the reference, whose partials are fp16: block3.rs:334-336): OR-ed into kvs_splits
 * (kvsplit 0x280) and into splits (combine 0x20), it makes the split kernel write its partial rows as f32 (512 B,
 * filling the fp32-sized rows the workspace already has) and the combine read them so. The split count is the low
 * 16 bits of either field; a launcher that follows the reference never sets bit 16. */
#define FMHA_KVS_F32_PARTIALS 0x10000u

/* Extensions of the full-sequence kernels' `flags` (0x280), no counterpart in the reference's MX kernels:
 *   FMHA_FLAG_CAUSAL    the bottom-right causal mask: key t visible to query i iff t <= i + SK - S;
 *   FMHA_FLAG_V_SEQ32   per-32-key V scales: ptr_v_descale (0x220) points to E8M0 bytes [B, ceil(SK/32), HK, 128]
 *                       (one per 32 keys per column, the layout of fmha_mxfp8_quantize_seq32) instead of one f32;
 *   FMHA_FLAG_SCALE     the softmax scale at 0x050 (f32, which the reference's MX kernels ignore: block3.rs:160) is
 *                       applied in the kernel: the scores are scale q.k (natural-log softmax), i.e. base-2 scores
 *                       c q.k with c = f32(scale log2 e), so Q must NOT carry the scale (quantise it with mul 1).
 *                       c = 2^e m (m in [1, 2)): 2^e joins the Q E8M0 exponents and S is multiplied by m
 *                       (the fp8pt family's way, block3.rs:160-173). c must be a positive normal f32.
 * For the KV split, FMHA_KVS_V_SEQ32 and FMHA_KVS_SCALE are OR-ed into kvs_splits (0x280) with the same meanings. */
#define FMHA_FLAG_CAUSAL 0x1u
#define FMHA_FLAG_V_SEQ32 0x2u
#define FMHA_FLAG_SCALE 0x4u
/* With FMHA_FLAG_CAUSAL: the causal q-tile pairing of the reference's causal kernels
 * (crates/amdgpu-stage/src/templates/grid.rs:94-111, causal_pair): block x runs query tiles x and T - 1 - x (the
 * second only when it is past x), T = ceil(S / rows), so every block does the same work; grid.x = ceil(T / 2).
 * The output is bit-identical to the unpaired launch (each tile is computed the same way). */
#define FMHA_FLAG_CAUSAL_PAIR 0x8u
#define FMHA_KVS_V_SEQ32 0x20000u
#define FMHA_KVS_SCALE 0x40000u

/* Byte sizes of the caller's allocations, checked by the validate calls
 * (the reference's BufferSizes, ..._vs128_abi.h:131-139). */
typedef struct fmha_mxfp8_buffer_sizes {
    uint64_t ptr_q, ptr_k, ptr_v, ptr_o;
    uint64_t ptr_q_descale, ptr_k_descale, ptr_v_descale;
    uint64_t ptr_ohat, ptr_lse;   /* KV split only */
} fmha_mxfp8_buffer_sizes;

/* ------------------------------------------------------------------------- */
/* Status codes                                                              */
/* ------------------------------------------------------------------------- */
enum {
    FMHA_OK = 0,
    FMHA_ERR_EXTENT = 1,      /* GV-HOST-EXTENT: a buffer is smaller than the contract */
    FMHA_ERR_KA_RANGE = 2,    /* GV-HOST-KA-RANGE: a kernarg field outside its range */
    FMHA_ERR_KA_IS = 3,       /* GV-HOST-KA-IS: a stride relation does not hold */
    FMHA_ERR_GRID = 4,        /* GV-HOST-GRID: grid does not match the shape */
    FMHA_ERR_SYM = 5,         /* GV-HOST-SYM: a host symbol outside its range */
    FMHA_ERR_PATH = 6,        /* unknown path / unsupported split count */
    FMHA_ERR_WORKSPACE = 7,   /* KV-split workspace missing or too small */
    FMHA_ERR_HIP = 8,         /* a HIP runtime call failed (message carries hipGetErrorString) */
    FMHA_ERR_NO_DEVICE = 9    /* no gfx950 device / code object failed to load */
};

/* Path identifiers of the dispatch. */
enum { FMHA_PATH_VS128 = 0, FMHA_PATH_T128 = 1, FMHA_PATH_KVSPLIT = 2 };

/* ------------------------------------------------------------------------- */
/* Host contract                                                             */
/* ------------------------------------------------------------------------- */

/* validate(): the reference's generated host contract, same rules and error
 * code prefixes. `err` (may be NULL) receives "GV-HOST-...: message".
 * Returns FMHA_OK or an FMHA_ERR_* code.
 * vs128: ..._vs128_abi.h:170-203; t128: ..._t128_abi.h (grid.x = ceil(S/128));
 * kvsplit: ..._kvsplit_abi.h (B, KL symbols, grid.z = B*splits);
 * combine: ..._kvsplit_combine8h_abi.h:56-65. */
int fmha_mxfp8_validate_vs128(const fmha_mxfp8_args* a, const fmha_mxfp8_buffer_sizes* sz,
                              uint32_t gx, uint32_t gy, uint32_t gz, int64_t HK, char* err, size_t errlen);
int fmha_mxfp8_validate_t128(const fmha_mxfp8_args* a, const fmha_mxfp8_buffer_sizes* sz,
                             uint32_t gx, uint32_t gy, uint32_t gz, int64_t HK, char* err, size_t errlen);
int fmha_mxfp8_validate_kvsplit(const fmha_mxfp8_kvsplit_args* a, const fmha_mxfp8_buffer_sizes* sz,
                                uint32_t gx, uint32_t gy, uint32_t gz, int64_t B, int64_t HK, int64_t KL,
                                char* err, size_t errlen);
int fmha_mxfp8_validate_combine(const fmha_mxfp8_combine_args* a, const fmha_mxfp8_buffer_sizes* sz,
                                uint32_t gx, uint32_t gy, uint32_t gz, char* err, size_t errlen);

/* Dispatch rule: mxfp8_prefill_path (crates/amdgpu-graph/src/dispatch.rs:494-511,
 * tests/gpu/ref_host.cpp:123-165). Returns FMHA_PATH_*; *splits = 0 unless KV split. */
int fmha_mxfp8_select_path(int64_t B, int64_t H, int64_t S, int64_t SK, int* splits);

/* Extension (no counterpart in the reference): 1 if fmha_fwd_hd128_mxfp8_auto runs the full-sequence `path`
 * (FMHA_PATH_VS128 or FMHA_PATH_T128) on the split-tile kernel fmha_fwd_hd128_mxfp8_v3_t128_split_tiles (128-row
 * blocks of 512 threads, the two wave groups splitting each tile's keys and merging at the end), else 0. t128: at
 * least 7 key tiles (4 with `causal`); below that the 256-thread fmha_fwd_hd128_mxfp8_v3_t128, which is faster there
 * and keeps the reference's order. vs128: the same, and a 256-row grid of at most 128 blocks unless `causal` (the
 * 128-row grid's causal q-tile pairing); such a half-chip grid below the threshold runs on the 256-thread t128
 * kernel. The split-tile order rounds differently from the reference's single stream per row; the path and its
 * recipe are the reference's. */
int fmha_mxfp8_uses_split_tiles(int path, int64_t B, int64_t H, int64_t S, int64_t SK, int causal);

/* Fill the kernarg fields derived from a packed [B,S,H,128] / [B,SK,HK,128]
 * layout (the values ref_host.cpp:342-360 and ops.py:114-118 write). */
void fmha_mxfp8_fill_args(fmha_mxfp8_args* a, void* o, const void* q, const void* k, const void* v,
                          const void* q_descale, const void* k_descale, const void* v_descale,
                          int B, int H, int HK, int S, int SK);

/* KV-split workspace bytes: fp32-sized partial rows + LSE (ref_host.cpp:146-149, ops.py:133-134). */
size_t fmha_mxfp8_workspace_bytes(int64_t B, int64_t H, int64_t S, int splits);

/* Extension (no counterpart in the reference): the number of partials per row that fmha_fwd_hd128_mxfp8_auto writes
 * for a KV split of `splits` chunks when its workspace holds them: each chunk's key range is divided into sub = 1, 2,
 * 4 or 8 consecutive ranges, sub doubling while the grid ((S + 255) / 256 x H x B x splits x sub blocks) stays within
 * the device's CU count and every range keeps at least 4 key tiles. Returns splits x sub (0 for invalid sizes). The
 * workspace for it is fmha_mxfp8_workspace_bytes(B, H, S, fmha_mxfp8_kv_partials(...)). */
int fmha_mxfp8_kv_partials(int64_t B, int64_t H, int64_t S, int64_t SK, int splits);

/* ------------------------------------------------------------------------- */
/* Launch                                                                    */
/* ------------------------------------------------------------------------- */
/* The generated launch() of each kernel (..._vs128_abi.h:204-209): validate is
 * NOT repeated here; the kernarg bytes are passed by
 * HIP_LAUNCH_PARAM_BUFFER_POINTER to hipModuleLaunchKernel on `stream`
 * (a hipStream_t, NULL = the null stream). Returns FMHA_OK or FMHA_ERR_HIP. */
int fmha_mxfp8_launch_vs128(const fmha_mxfp8_args* a, uint32_t gx, uint32_t gy, uint32_t gz, void* stream);
int fmha_mxfp8_launch_t128(const fmha_mxfp8_args* a, uint32_t gx, uint32_t gy, uint32_t gz, void* stream);
/* Extension (no counterpart in the reference): the split-tile kernel fmha_fwd_hd128_mxfp8_v3_t128_split_tiles on
 * t128's grid (ceil(S/128), H, B) and kernarg layout, 512 threads; the two wave groups split each key tile and merge
 * at the end (the order fmha_mxfp8_uses_split_tiles names). fmha_fwd_hd128_mxfp8_auto runs it for t128's shapes with
 * at least 7 key tiles (4 with the causal mask) and for vs128's shapes whose 256-row grid has at most 128 blocks
 * (from the same key-tile counts). */
int fmha_mxfp8_launch_t128_split_tiles(const fmha_mxfp8_args* a, uint32_t gx, uint32_t gy, uint32_t gz, void* stream);
int fmha_mxfp8_launch_kvsplit(const fmha_mxfp8_kvsplit_args* a, uint32_t gx, uint32_t gy, uint32_t gz, void* stream);
int fmha_mxfp8_launch_combine(const fmha_mxfp8_combine_args* a, uint32_t gx, void* stream);
/* Extension (no counterpart in the reference): the same merge on fmha_fwd_hd128_mxfp8_v3_kvsplit_combine_wide, which
 * spreads each row's splits over a block's 4 waves (quarters merged in order): 64 groups of 8 outputs per block, grid
 * gx = ceil(rows_total x 16 / 64), 256 threads. Same arguments and rules as the combine; the one-call entry runs it
 * for more than 8 partials per row. */
int fmha_mxfp8_launch_combine_wide(const fmha_mxfp8_combine_args* a, uint32_t gx, void* stream);

/* Problem description of the one-call entry. All pointers are device pointers
 * to packed tensors (layouts in fmha_mxfp8_args). */
typedef struct fmha_mxfp8_params {
    void* o;
    const void* q; const void* k; const void* v;
    const void* q_descale; const void* k_descale; const void* v_descale;
    void* lse;                 /* optional [B,H,S] f32 natural-log LSE (vs128/t128 only), NULL = none */
    uint64_t bytes_q, bytes_k, bytes_v, bytes_o;
    uint64_t bytes_q_descale, bytes_k_descale, bytes_v_descale;
    int32_t B, H, HK, S, SK;
    int32_t path;              /* -1 = auto (dispatch rule), else FMHA_PATH_* */
    int32_t splits;            /* KV split chunks when path == FMHA_PATH_KVSPLIT (2, 4 or 8; 0 = 4) */
    int32_t causal;            /* 0 = the reference semantics; 1 = bottom-right causal mask (extension) */
    int32_t f32_partials;      /* KV split only: 0 = fp16 partial rows (the reference's); 1 = f32 (extension) */
    int32_t v_seq32;           /* 0 = v_descale is one f32 (the reference's); 1 = E8M0 per 32 keys per column (extension) */
    float softmax_scale;       /* 0 = the reference's convention (the scale is folded into Q before quantisation);
                                  > 0 = applied in the kernel (FMHA_FLAG_SCALE / FMHA_KVS_SCALE, extension) */
    int32_t no_check;          /* 0 = run the validate rules before launching (the default); 1 = skip them, as the
                                  reference op's check=False does (python/amdgpu_jit/ops.py:88): the caller then
                                  vouches for the buffer extents and strides */
    int32_t causal_pair;       /* causal only (extension): 0 = the causal q-tile pairing (FMHA_FLAG_CAUSAL_PAIR) when
                                  the unpaired grid has more blocks than the device has CUs; 1 = always; 2 = never */
    int32_t kv_fill;           /* KV split only (extension): 0 = each chunk spread over the blocks that
                                  fmha_mxfp8_kv_partials names, as far as the workspace holds their partials;
                                  1 = the reference's chunks only (one block per chunk and query tile) */
    uint32_t* ws_turn;         /* KV split only (extension), optional: a turn word the caller owns (host memory). With a
                                  workspace of several slots the call uses slot *ws_turn % slots and increments the
                                  word; NULL = slot 0. Calls that share a word take the slots in turn; callers with
                                  their own words (and workspaces) never affect each other's slots. */
    int32_t* partials_out;     /* optional output (extension): the KV split's partials per row that ran (the chunks
                                  times the KV fill; 0 off the KV split) */
} fmha_mxfp8_params;

/* fmha_fwd_hd128_mxfp8_auto: dispatch + validate + launch (+ combine), all on
 * `stream`, no host synchronisation. `workspace` (device, >= the value of
 * fmha_mxfp8_workspace_bytes for the partials that run, p->partials_out) is
 * needed only when the KV split runs; it may be NULL otherwise. On return
 * *path_out / *splits_out (may be NULL) name what ran: the path and, for the
 * KV split, its chunk count (2, 4 or 8), as the reference op returns them.
 * Mirrors python/amdgpu_jit/ops.py:88-143. The library keeps no mutable state
 * between calls (the compiled-module and CU-count caches aside).
 * Extension: a workspace of k >= 2 times that size (each copy rounded up to 256 B) is used as min(k,
 * FMHA_WORKSPACE_SLOTS) slots taken in turn through the caller's p->ws_turn word, so that a call's split kernel does
 * not write the lines the previous call's combine has just read (on MI355X that costs up to a quarter of the call:
 * B1H8S2048 with 4 splits runs 25.6 us per call on one slot, 19.1 us on four). The minimum size, or no turn word,
 * keeps the reference's behaviour. */
#define FMHA_WORKSPACE_SLOTS 4u
int fmha_fwd_hd128_mxfp8_auto(const fmha_mxfp8_params* p, void* workspace, size_t workspace_bytes,
                              void* stream, int* path_out, int* splits_out, char* err, size_t errlen);

/* Allocation-free variant of fmha_fwd_hd128_mxfp8_auto. No counterpart in the reference: it is for callers that
 * cannot allocate device memory or pass a workspace (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). The KV split's workspace is a device array of FMHA_NOALLOC_SCRATCH_BYTES inside the library
 * instead of a caller's buffer, one per device, held until the process ends; a shape whose split needs more is
 * rejected with FMHA_ERR_WORKSPACE. The largest workspace the auto dispatch asks for is 2 splits x 32768 rows x 516 B
 * (blocks256 <= 128 bounds B S H to 32768): exactly this size; the KV fill and the workspace slots (taken in turn
 * through p->ws_turn when the caller passes one, else slot 0) use as much of it as it holds. The first call on a
 * device looks the array up and loads
 * the code objects (fmha_mxfp8_init); later calls call no allocating routine and no hipMalloc/hipFree. Calls on one
 * device share its array: calls that overlap on one device (unordered streams) race. Otherwise identical to
 * fmha_fwd_hd128_mxfp8_auto (same params, rules, errors and kernels). */
#define FMHA_NOALLOC_SCRATCH_BYTES 33816576u
int fmha_fwd_hd128_mxfp8_auto_noalloc(const fmha_mxfp8_params* p, void* stream, int* path_out, int* splits_out,
                                      char* err, size_t errlen);

/* Loads the embedded code object on the current device (done lazily by the
 * launch calls; exposed so a caller can fail early). */
int fmha_mxfp8_init(char* err, size_t errlen);

/* Library version string. */
const char* fmha_mxfp8_version(void);

#ifdef __cplusplus
}
#endif
#endif /* FMHA_MXFP8_H */
