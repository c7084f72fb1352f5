/*
 * mxfp8_oracle.h - CPU restatement of the reference's MXFP8 FMHA-forward path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (amdgpu_rustdsl_amd/,
 * include/) links, loads or calls this code; only tests/, the smoke check and
 * bench.py's cpu_baseline leg use it, and only as the checker / the timed CPU
 * baseline, never as the thing measured or shipped.
 *
 * Contents and the reference code each part restates:
 *   mxo_e4m3_decode / mxo_e4m3_encode   tests/gpu/ref_host.cpp:26-33, 216-228
 *   mxo_generate                        tests/gpu/ref_host.cpp:183-263 (REF_DATA lcg | uniform | normal)
 *   mxo_quant_rows_bf16 / _tensor_bf16 /
 *   mxo_quant_seq32_bf16                the generator's quantisation rule (ref_host.cpp:239-251) applied to
 *                                       given bf16 values (the checker of the on-GPU quantisers)
 *   mxo_select_path                     crates/amdgpu-graph/src/dispatch.rs:494-511
 *   mxo_split_range                     crates/amdgpu-stage/src/components.rs:58-74
 *   mxo_check_fp64                      tests/gpu/ref_host.cpp:436-471
 *   mxo_attention_fp32                  the CPU baseline (fp32 attention on dequantised inputs)
 *   mxo_emulate                         the reference kernels' recipe, bit-level model:
 *       crates/amdgpu-tile/src/softmax.rs:67-243 (two-word reference, eager/lazy rollback),
 *       crates/amdgpu-tile/src/reduce.rs:66-113 (pknorm exp2, LUT correction, scaled fp8 P),
 *       crates/amdgpu-stage/src/attention/state.rs:75-83 (recipe copy, output scale),
 *       crates/amdgpu-stage/src/attention/block3.rs:291-356 + softmax.rs:308-322 (split partials),
 *       crates/amdgpu-tile/src/epilogue.rs:89-167 (combine)
 */
#ifndef MXFP8_ORACLE_H
#define MXFP8_ORACLE_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

typedef struct mxo_problem {
    int B, H, HK, S, SK;
    const uint8_t* q;   /* [B,S,H,128] e4m3 */
    const uint8_t* k;   /* [B,SK,HK,128] */
    const uint8_t* v;   /* [B,SK,HK,128] */
    const uint8_t* qs;  /* [B,S,H,4] E8M0 */
    const uint8_t* ks;  /* [B,SK,HK,4] E8M0 */
    float vdescale;
    int causal;         /* bottom-right causal mask: key t visible for query i iff t <= i + SK - S */
    const uint8_t* vs32;/* extension: NULL = one f32 V descale (vdescale, the reference's); else E8M0 V scales
                           [B, ceil(SK/32), HK, 128], one per 32 keys per column, and vdescale is not used */
    float qk_scale;     /* extension: 0 = the reference's convention (the softmax scale is folded into Q, scores are
                           base-2 q.k); > 0 = the kernel applies it: base-2 scores c q.k with c = f32(qk_scale log2 e) */
} mxo_problem;

typedef struct mxo_check_result {
    uint64_t checked, bad;
    double worst_err, mean_err, max_ref;
} mxo_check_result;

/* e4m3 byte -> value (NaN encoding 0x7F/0xFF decodes to 0, as ref_host.cpp:28). */
double mxo_e4m3_decode(uint8_t b);
/* Round-to-nearest-even e4m3 encoder saturating at 448 (ref_host.cpp:216-228). */
uint8_t mxo_e4m3_encode_sat(float x);
/* The gfx950 scaled conversion v_cvt_scalef32_pk_fp8_bf16 on one bf16 value:
 * e4m3(RNE(bf16 / scale)), |x| > 464 -> NaN byte (0x7F | sign); NaN -> 0xFF. */
uint8_t mxo_cvt_bf16_fp8(uint16_t bf16, float scale);
/* v_cvt_pknorm_u16_f32: round-to-nearest-even of 65535 * clamp(x, 0, 1). */
uint16_t mxo_pknorm_u16(float x);
float mxo_f16_to_f32(uint16_t h);
uint16_t mxo_f32_to_f16(float f);     /* RNE */
uint16_t mxo_f32_to_bf16(float f);    /* RNE */
float mxo_bf16_to_f32(uint16_t b);

/* Sizes of the generator's buffers (descale buffers include the zeroed slack
 * ref_host.cpp:196-198 appends). */
size_t mxo_qs_bytes(int B, int H, int S);
size_t mxo_ks_bytes(int B, int H, int HK, int SK);

/* Input generator. mode: 0 = lcg (palette), 1 = uniform, 2 = normal.
 * Buffers: q [B*S*H*128], k/v [B*SK*HK*128], qs [mxo_qs_bytes], ks [mxo_ks_bytes].
 * Returns the V descale (1.0 for lcg/uniform). seed_mix = 0 reproduces
 * ref_host.cpp bit for bit; a non-zero value is xor-ed into both seeds
 * (a second, independent input set). */
float mxo_generate(int mode, int B, int H, int HK, int S, int SK, uint64_t seed_mix,
                   uint8_t* q, uint8_t* k, uint8_t* v, uint8_t* qs, uint8_t* ks);

/* Dispatch: returns 0 vs128, 1 t128, 2 kvsplit; *splits set for kvsplit. */
/* x [rows,128] bf16 -> q [rows,128] e4m3 + sc [rows,4] E8M0; x is multiplied by `mul` in f32 first. */
void mxo_quant_rows_bf16(const uint16_t* x, long rows, float mul, uint8_t* q, uint8_t* sc);
/* x [n] bf16 -> q [n] e4m3; returns the f32 descale amax / 448. */
float mxo_quant_tensor_bf16(const uint16_t* x, long n, uint8_t* q);
/* x [B,SK,HK,128] bf16 -> q (same shape) e4m3 + sc [B,ceil(SK/32),HK,128] E8M0 (per 32 keys per column). */
void mxo_quant_seq32_bf16(const uint16_t* x, int B, int SK, int HK, uint8_t* q, uint8_t* sc);

int mxo_select_path(long B, long H, long S, long SK, int* splits);
/* KV-split range of split `s`: [*key_lo, *key_lo + *kv_eff). */
void mxo_split_range(int SK, int splits, int s, int* key_lo, int* kv_eff);

/* fp64 attention check of a bf16 output [B,S,H,128] on the first `rows` query
 * rows of every (b, h) (ref_host.cpp:436-471; scale ln 2). threads <= 0: all cores. */
mxo_check_result mxo_check_fp64(const mxo_problem* p, const uint16_t* out_bf16, int rows, int threads);
/* The same over the query rows row_list[0 .. nrows) of every (b, h) (each in [0, S), any order). */
mxo_check_result mxo_check_fp64_rows(const mxo_problem* p, const uint16_t* out_bf16, const int* row_list, int nrows, int threads);

/* fp32 attention on the dequantised inputs for rows [0, rows) of every (b,h)
 * (rows <= 0: all), result into out_f32 [B,S,H,128] (may be NULL: compute only).
 * Returns wall seconds. threads <= 0: all cores. */
double mxo_attention_fp32(const mxo_problem* p, int rows, float* out_f32, int threads);

/* Bit-level model of the reference kernels for the first `rows` rows of every
 * (b,h) (rows <= 0: all). splits == 0: the full-sequence kernels (_vs128 /
 * _t128, identical numerics); splits in {2,4,8}: _kvsplit + _kvsplit_combine8h.
 * out_bf16 [B,S,H,128]: only the emulated rows are written.
 * If ohat_f16 / lse_f32 are non-NULL (splits > 0) the partials are written in
 * the kernel's layout: row index split*rows_total + (b*S + row)*H + h. */
void mxo_emulate(const mxo_problem* p, int splits, int rows, uint16_t* out_bf16,
                 uint16_t* ohat_f16, float* lse_f32, int threads);

/* The combine kernel's arithmetic on given partials (epilogue.rs:89-167). */
void mxo_combine(const uint16_t* ohat_f16, const float* lse, uint16_t* out_bf16, long rows_total, int splits);

/* Extension (no reference counterpart): mxo_emulate with the KV split's partial rows kept in f32 when f32_partials
 * (ohat then receives f32 rows), and the combine on f32 partial rows. split_tiles: the library's split-tile order
 * (two 64-key streams per tile, merged; non-LUT recipe only) for KV-split blocks of at most 128 query rows, and,
 * with splits = 0, for every row (the t128 path's split-tile kernel).
 * mxo_emulate is mxo_emulate_ex(..., 0, 0, ...). */
/* at most MXO_MAX_SPLITS splits (more: nothing is written) */
#define MXO_MAX_SPLITS 64
void mxo_emulate_ex(const mxo_problem* p, int splits, int rows, uint16_t* out_bf16, void* ohat, float* lse_f32,
                    int f32_partials, int split_tiles, int threads);
/* mxo_emulate_ex (no partials out) over the query rows row_list[0 .. nrows) of every (b, h). */
void mxo_emulate_rows(const mxo_problem* p, int splits, const int* row_list, int nrows, uint16_t* out_bf16, int f32_partials,
                      int split_tiles, int threads);
void mxo_combine_f32(const float* ohat_f32, const float* lse, uint16_t* out_bf16, long rows_total, int splits);

#ifdef __cplusplus
}
#endif
#endif
