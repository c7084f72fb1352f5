// fmha_host.cpp - host side of the MXFP8 FMHA forward: the C ABI of include/fmha_mxfp8.h.
//
// The host contract (validate), the dispatch rule, the kernarg filling and the launches through
// hipModuleLaunchKernel with HIP_LAUNCH_PARAM_BUFFER_POINTER, exactly the way the reference's generated
// headers launch its kernels (tests/gpu/generated/fmha_fwd_hd128_mxfp8_v3_vs128_abi.h:204-209). The gfx950
// code object (fmha_kernels.hip) is embedded in this library at build time and loaded once per device with
// hipModuleLoadData. No function allocates device memory; the KV-split workspace is the caller's.

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <atomic>
#include <cstdlib>

#include "../../include/fmha_mxfp8.h"
#include "module_cache.h"

static_assert(sizeof(fmha_mxfp8_args) == 656, "kernarg size (vs128_abi.h:126)");
static_assert(sizeof(fmha_mxfp8_params) == 192, "params layout (lib.py mirrors it)");
static_assert(offsetof(fmha_mxfp8_args, ptr_o) == 0x000, "ptr_o");
static_assert(offsetof(fmha_mxfp8_args, ptr_q) == 0x010, "ptr_q");
static_assert(offsetof(fmha_mxfp8_args, ptr_k) == 0x020, "ptr_k");
static_assert(offsetof(fmha_mxfp8_args, ptr_v) == 0x030, "ptr_v");
static_assert(offsetof(fmha_mxfp8_args, ptr_lse) == 0x040, "ptr_lse");
static_assert(offsetof(fmha_mxfp8_args, softmax_scale) == 0x050, "scale");
static_assert(offsetof(fmha_mxfp8_args, s_seq_len) == 0x060, "s_seq_len");
static_assert(offsetof(fmha_mxfp8_args, s_Seqs) == 0x070, "s_Seqs");
static_assert(offsetof(fmha_mxfp8_args, s_Hs) == 0x090, "s_Hs");
static_assert(offsetof(fmha_mxfp8_args, s_Bs) == 0x0A0, "s_Bs");
static_assert(offsetof(fmha_mxfp8_args, s_gqa) == 0x0B0, "s_gqa");
static_assert(offsetof(fmha_mxfp8_args, s_k_Seqs) == 0x0C0, "s_k_Seqs");
static_assert(offsetof(fmha_mxfp8_args, s_k_Hs) == 0x0D0, "s_k_Hs");
static_assert(offsetof(fmha_mxfp8_args, s_k_Bs) == 0x0E0, "s_k_Bs");
static_assert(offsetof(fmha_mxfp8_args, opt) == 0x0F0, "opt");
static_assert(offsetof(fmha_mxfp8_args, s_kv_seq_len) == 0x110, "s_kv_seq_len");
static_assert(offsetof(fmha_mxfp8_args, s_q_head_num) == 0x140, "s_q_head_num");
static_assert(offsetof(fmha_mxfp8_args, s_v_Seqs) == 0x150, "s_v_Seqs");
static_assert(offsetof(fmha_mxfp8_args, s_v_Hs) == 0x160, "s_v_Hs");
static_assert(offsetof(fmha_mxfp8_args, s_v_Bs) == 0x170, "s_v_Bs");
static_assert(offsetof(fmha_mxfp8_args, s_o_Seqs) == 0x180, "s_o_Seqs");
static_assert(offsetof(fmha_mxfp8_args, s_o_Hs) == 0x190, "s_o_Hs");
static_assert(offsetof(fmha_mxfp8_args, s_o_Bs) == 0x1A0, "s_o_Bs");
static_assert(offsetof(fmha_mxfp8_args, ptr_q_descale) == 0x200, "ptr_q_descale");
static_assert(offsetof(fmha_mxfp8_args, ptr_k_descale) == 0x210, "ptr_k_descale");
static_assert(offsetof(fmha_mxfp8_args, ptr_v_descale) == 0x220, "ptr_v_descale");
static_assert(offsetof(fmha_mxfp8_args, s_descale_q_Bs) == 0x230, "s_descale_q_Bs");
static_assert(offsetof(fmha_mxfp8_args, s_descale_q_Hs) == 0x240, "s_descale_q_Hs");
static_assert(offsetof(fmha_mxfp8_args, s_descale_k_Bs) == 0x250, "s_descale_k_Bs");
static_assert(offsetof(fmha_mxfp8_args, s_descale_k_Hs) == 0x260, "s_descale_k_Hs");
static_assert(offsetof(fmha_mxfp8_args, flags) == 0x280, "flags / abi_tail");
static_assert(sizeof(fmha_mxfp8_kvsplit_args) == 648, "kvsplit kernarg size (kvsplit_abi.h:136)");
static_assert(offsetof(fmha_mxfp8_kvsplit_args, ptr_ohat) == 0x270, "ptr_ohat");
static_assert(offsetof(fmha_mxfp8_kvsplit_args, ptr_lse) == 0x278, "ptr_lse");
static_assert(offsetof(fmha_mxfp8_kvsplit_args, kvs_splits) == 0x280, "kvs_splits");
static_assert(offsetof(fmha_mxfp8_kvsplit_args, kvs_rows_total) == 0x284, "kvs_rows_total");
static_assert(sizeof(fmha_mxfp8_combine_args) == 36, "combine kernarg size (combine8h_abi.h:34)");
static_assert(offsetof(fmha_mxfp8_combine_args, rows_total) == 0x18, "rows_total");
static_assert(offsetof(fmha_mxfp8_combine_args, splits) == 0x20, "splits");

// The code object, embedded by the build (FMHA_HSACO_PATH names the file built from fmha_kernels.hip).
#ifndef FMHA_HSACO_PATH
#error "FMHA_HSACO_PATH must name the gfx950 code object built from fmha_kernels.hip"
#endif
asm(".section .rodata.fmha_hsaco,\"a\",@progbits\n"
    ".balign 4096\n"
    ".global fmha_mxfp8_hsaco_begin\n"
    "fmha_mxfp8_hsaco_begin:\n"
    ".incbin \"" FMHA_HSACO_PATH "\"\n"
    ".global fmha_mxfp8_hsaco_end\n"
    "fmha_mxfp8_hsaco_end:\n"
    ".previous\n");
extern "C" const unsigned char fmha_mxfp8_hsaco_begin[];
extern "C" const unsigned char fmha_mxfp8_hsaco_end[];

namespace {

using fmha_internal::fail;
using fmha_internal::set_err;

const char* const kKernelNames[10] = {
    "fmha_fwd_hd128_mxfp8_v3_vs128",
    "fmha_fwd_hd128_mxfp8_v3_t128",
    "fmha_fwd_hd128_mxfp8_v3_kvsplit",
    "fmha_fwd_hd128_mxfp8_v3_kvsplit_combine8h",
    // extension kernels: the softmax scale at 0x050 applied in the kernel (FMHA_FLAG_SCALE / FMHA_KVS_SCALE)
    "fmha_fwd_hd128_mxfp8_v3_vs128_scaled",
    "fmha_fwd_hd128_mxfp8_v3_t128_scaled",
    "fmha_fwd_hd128_mxfp8_v3_kvsplit_scaled",
    // extension kernels: t128's grid with 512 threads, the two wave groups splitting each tile's keys
    "fmha_fwd_hd128_mxfp8_v3_t128_split_tiles",
    "fmha_fwd_hd128_mxfp8_v3_t128_split_tiles_scaled",
    // extension kernel: the combine with the splits spread over 4 waves (more than 8 partials per row)
    "fmha_fwd_hd128_mxfp8_v3_kvsplit_combine_wide",
};
enum { K_VS128 = 0, K_T128 = 1, K_KVSPLIT = 2, K_COMBINE = 3, K_VS128_SC = 4, K_T128_SC = 5, K_KVSPLIT_SC = 6, K_T128ST = 7,
       K_T128ST_SC = 8, K_COMBINE_WIDE = 9 };

// The 128-row grids (t128's shapes, and vs128's half-chip and causal ones below) run on the split-tile kernel (512
// threads) from 7 key tiles on, and on the one-wave-per-SIMD kernel (256 threads, the reference's order) below that:
// with 4 to 6 key tiles the single-wave kernel is faster (measured on MI355X, us: B1H8S512 9.11 against 9.92,
// B1H8S1024 SK768 11.52 against 11.73, B4H8S512 9.45 against 10.28, B8H8S512 9.78 against 10.75; at SK1024 13.78
// against 13.16), and with fewer than 4 (the LUT recipe, state.rs:75-77) it keeps the reference's order. Causal
// shapes take the split-tile kernel from 4 key tiles on (unpaired it is ahead: B1H8S1024 causal 13.56 against 14.45)
// except on grids the causal q-tile pairing halves (more 128-row blocks than CUs) with at most 8 key tiles, where the
// single-wave kernel runs each pair faster (B16H8S512 15.13 against 17.07, B8H8S768 16.94 against 18.34, B8H8S1024
// 19.45 against 20.13; at 16 tiles, B4H8S2048, 28.37 against 26.63). The choice does not depend on the causal_pair
// field, so a forced pairing gives the same kernel, and so the same bits, as the automatic one.
int cu_count();
bool use_split_tiles(int64_t B, int64_t H, int64_t S, int64_t SK, bool causal) {
    const int64_t tiles = (SK + 127) / 128;
    if (!causal) return tiles >= 7;
    if (tiles < 4) return false;
    return !(tiles <= 8 && (S + 127) / 128 * H * B > (int64_t)cu_count());
}

// The one-call entry also runs the vs128 path on the 128-row grid when its 256-row grid holds at most 128 blocks (half
// of the 256 CUs or fewer): there the same shape fills twice the CUs. Causal (extension): always from 4 key tiles on,
// so that the 128-row grid's causal q-tile pairing is available past one wave of blocks. The kernel is chosen as for
// t128 (above). Below the split-tile threshold the 256-thread t128 kernel gives the vs128 kernel's order and bits
// (both take every tile whole) on twice the blocks; measured with the LUT recipe at B4H8S1024 SK256, B2H8S2048 SK384
// and B1H8S4096 SK128: 10.4 / 12.6 / 7.7 us against 11.9 / 14.3 / 9.5 (above 128 blocks of 256 rows the vs128 kernel
// stays ahead: B8H8S2048 SK256 25.4 against 36.4 us). The direct vs128 launcher keeps the 256-row kernel its grid names.
bool vs128_on_128row_grid(int64_t B, int64_t H, int64_t S, int64_t SK, bool causal) {
    return (S + 255) / 256 * H * B <= 128 || (causal && (SK + 127) / 128 >= 4);
}

fmha_internal::ModuleCache<10> g_fmha(fmha_mxfp8_hsaco_begin, fmha_mxfp8_hsaco_end, kKernelNames);

int get_functions(hipFunction_t** out, char* err, size_t errlen) { return g_fmha.get(out, err, errlen); }

int launch_raw(int which, const void* args, size_t nbytes, uint32_t gx, uint32_t gy, uint32_t gz, uint32_t block,
               void* stream, char* err, size_t errlen) {
    return g_fmha.launch(which, args, nbytes, gx, gy, gz, block, stream, err, errlen);
}

typedef long long i64;

// The 0x000-0x26F rules shared by vs128 / t128 / kvsplit (vs128_abi.h:170-203), in the reference's four groups
// and order: buffer extents, kernarg ranges, kernarg relations, grid. `B` is grid.z for the single-kernel launches
// and the host symbol B for the KV split (kvsplit_abi.h).
// v_seq32: the per-32-key V-scale extension, whose ptr_v_descale holds E8M0 [B, ceil(SK/32), HK, 128]
int rules_extent(const fmha_mxfp8_args& a, const fmha_mxfp8_buffer_sizes& sz, i64 B, bool v_seq32, char* err, size_t errlen) {
    const i64 H = a.s_q_head_num;
    if (sz.ptr_q < (uint64_t)(B * (i64)a.s_Bs)) return fail(err, errlen, FMHA_ERR_EXTENT, "GV-HOST-EXTENT", "ptr_q: buffer ptr_q smaller than declared allocation");
    if (sz.ptr_k < (uint64_t)(B * (i64)a.s_k_Bs)) return fail(err, errlen, FMHA_ERR_EXTENT, "GV-HOST-EXTENT", "ptr_k: buffer ptr_k smaller than declared allocation");
    if (sz.ptr_v < (uint64_t)(B * (i64)a.s_v_Bs)) return fail(err, errlen, FMHA_ERR_EXTENT, "GV-HOST-EXTENT", "ptr_v: buffer ptr_v smaller than declared allocation");
    if (sz.ptr_o < (uint64_t)(B * (i64)a.s_o_Bs)) return fail(err, errlen, FMHA_ERR_EXTENT, "GV-HOST-EXTENT", "ptr_o: buffer ptr_o smaller than declared allocation");
    if (sz.ptr_q_descale < (uint64_t)(B * (i64)a.s_descale_q_Bs + 2048LL * H))
        return fail(err, errlen, FMHA_ERR_EXTENT, "GV-HOST-EXTENT", "ptr_q_descale: buffer ptr_q_descale smaller than declared allocation");
    if (sz.ptr_k_descale < (uint64_t)(B * (i64)a.s_descale_k_Bs + 2560LL * H))
        return fail(err, errlen, FMHA_ERR_EXTENT, "GV-HOST-EXTENT", "ptr_k_descale: buffer ptr_k_descale smaller than declared allocation");
    const uint64_t vd_need = v_seq32 ? (uint64_t)(B * (((i64)a.s_kv_seq_len + 31) / 32) * (i64)a.s_k_Seqs) : 4096ull;
    if (sz.ptr_v_descale < vd_need) return fail(err, errlen, FMHA_ERR_EXTENT, "GV-HOST-EXTENT", "ptr_v_descale: buffer ptr_v_descale smaller than declared allocation");
    return FMHA_OK;
}

int rules_range(const fmha_mxfp8_args& a, char* err, size_t errlen) {
    const i64 gqa = a.s_gqa;
    if (gqa < 1 || gqa > 16) return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "ka(0xB0) outside contract");
    if (a.s_seq_len < 1) return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "ka(0x60) outside contract");
    if (a.s_kv_seq_len < 1) return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "ka(0x110) outside contract");
    if (a.s_Hs != 128) return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "ka(0x90) outside contract");
    if (a.s_k_Hs != 128) return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "ka(0xD0) outside contract");
    if (a.s_v_Hs != 128) return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "ka(0x160) outside contract");
    if (a.s_o_Hs != 256) return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "ka(0x190) outside contract");
    if (a.s_descale_q_Hs != 4) return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "ka(0x240) outside contract");
    if (a.s_descale_k_Hs != 4) return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "ka(0x260) outside contract");
    return FMHA_OK;
}

int rules_is(const fmha_mxfp8_args& a, i64 HK, char* err, size_t errlen) {
    const i64 S = a.s_seq_len, SK = a.s_kv_seq_len, H = a.s_q_head_num;
    if (H != HK * (i64)a.s_gqa) return fail(err, errlen, FMHA_ERR_KA_IS, "GV-HOST-KA-IS", "ka(0x140) relation failed");
    if ((i64)a.s_Seqs != H * 128) return fail(err, errlen, FMHA_ERR_KA_IS, "GV-HOST-KA-IS", "ka(0x70) relation failed");
    if ((i64)a.s_Bs != S * (i64)a.s_Seqs) return fail(err, errlen, FMHA_ERR_KA_IS, "GV-HOST-KA-IS", "ka(0xA0) relation failed");
    if ((i64)a.s_k_Seqs != HK * 128) return fail(err, errlen, FMHA_ERR_KA_IS, "GV-HOST-KA-IS", "ka(0xC0) relation failed");
    if ((i64)a.s_k_Bs != SK * (i64)a.s_k_Seqs) return fail(err, errlen, FMHA_ERR_KA_IS, "GV-HOST-KA-IS", "ka(0xE0) relation failed");
    if (a.s_v_Seqs != a.s_k_Seqs) return fail(err, errlen, FMHA_ERR_KA_IS, "GV-HOST-KA-IS", "ka(0x150) relation failed");
    if (a.s_v_Bs != a.s_k_Bs) return fail(err, errlen, FMHA_ERR_KA_IS, "GV-HOST-KA-IS", "ka(0x170) relation failed");
    if ((i64)a.s_o_Seqs != H * 256) return fail(err, errlen, FMHA_ERR_KA_IS, "GV-HOST-KA-IS", "ka(0x180) relation failed");
    if ((i64)a.s_o_Bs != S * (i64)a.s_o_Seqs) return fail(err, errlen, FMHA_ERR_KA_IS, "GV-HOST-KA-IS", "ka(0x1A0) relation failed");
    if ((i64)a.s_descale_q_Bs != S * H * 4) return fail(err, errlen, FMHA_ERR_KA_IS, "GV-HOST-KA-IS", "ka(0x230) relation failed");
    if ((i64)a.s_descale_k_Bs != SK * HK * 4) return fail(err, errlen, FMHA_ERR_KA_IS, "GV-HOST-KA-IS", "ka(0x250) relation failed");
    return FMHA_OK;
}

int rules_grid(const fmha_mxfp8_args& a, uint32_t gx, uint32_t gy, int rows_per_block, char* err, size_t errlen) {
    if ((i64)gy != (i64)a.s_q_head_num) return fail(err, errlen, FMHA_ERR_GRID, "GV-HOST-GRID", "grid axis 1 relation failed");
    i64 want = ((i64)a.s_seq_len + rows_per_block - 1) / rows_per_block;
    if (a.flags & FMHA_FLAG_CAUSAL_PAIR) want = (want + 1) / 2;   // the causal q-tile pairing: two tiles per block
    if ((i64)gx != want) return fail(err, errlen, FMHA_ERR_GRID, "GV-HOST-GRID", "grid axis 0 relation failed");
    return FMHA_OK;
}

// Compute units of the current device (the causal pairing pays off only when the unpaired grid exceeds them), cached
// FMHA_MXFP8_CU_COUNT (a positive integer) replaces the device's count: the CU-dependent rules (the KV fill, the
// causal pairing, the causal split-tile choice) and so the output bits can then be checked for another part's count,
// also on a machine without a GPU.
int cu_count() {
    static const int env = [] {
        const char* e = std::getenv("FMHA_MXFP8_CU_COUNT");
        return e ? std::atoi(e) : 0;
    }();
    if (env > 0) return env;
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n <= 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cache[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

// The in-kernel softmax scale (FMHA_FLAG_SCALE / FMHA_KVS_SCALE): c = f32(scale log2 e) must be a positive normal f32
// (its exponent then splits off exactly, and the Q scale exponents shift by it)
bool scale_ok(float scale) {
    const float c = scale * 1.44269504088896340736f;
    return std::isfinite(c) && std::isnormal(c) && c > 0.0f;
}
int rules_scale(const fmha_mxfp8_args& a, bool on, char* err, size_t errlen) {
    float scale;
    std::memcpy(&scale, &a.softmax_scale, 4);
    if (on && !scale_ok(scale))
        return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "ka(0x50) outside contract (softmax scale)");
    return FMHA_OK;
}

int validate_base(const fmha_mxfp8_args& a, const fmha_mxfp8_buffer_sizes& sz, uint32_t gx, uint32_t gy, i64 B, i64 HK,
                  int rows_per_block, char* err, size_t errlen) {
    int rc;
    if ((rc = rules_extent(a, sz, B, (a.flags & FMHA_FLAG_V_SEQ32) != 0, err, errlen)) != FMHA_OK) return rc;
    if ((rc = rules_range(a, err, errlen)) != FMHA_OK) return rc;
    if ((a.flags & ~(FMHA_FLAG_CAUSAL | FMHA_FLAG_V_SEQ32 | FMHA_FLAG_SCALE | FMHA_FLAG_CAUSAL_PAIR)) != 0 ||
        ((a.flags & FMHA_FLAG_CAUSAL_PAIR) && !(a.flags & FMHA_FLAG_CAUSAL)))
        return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "ka(0x280) outside contract");
    if ((rc = rules_scale(a, (a.flags & FMHA_FLAG_SCALE) != 0, err, errlen)) != FMHA_OK) return rc;
    if ((rc = rules_is(a, HK, err, errlen)) != FMHA_OK) return rc;
    return rules_grid(a, gx, gy, rows_per_block, err, errlen);
}

bool empty_split(i64 SK, i64 splits) {
    const i64 ntiles = (SK + 127) / 128;
    const i64 tps = (ntiles + splits - 1) / splits;
    return !((splits - 1) * tps < ntiles);
}

// KV-split fill (extension): the reference's `splits` chunks, each divided into `sub` consecutive key ranges, so that
// a grid of few blocks fills the CUs. sub doubles (up to 8) while the grid stays within the CU count and every range
// keeps at least 4 key tiles (the recipe of the reference's splits, which have at least 4). The combine merges the
// splits x sub partials.
i64 kv_fill(i64 B, i64 H, i64 S, i64 SK, i64 splits) {
    const i64 blocks = (S + 255) / 256 * H * B * splits, tiles = (SK + 127) / 128;
    i64 sub = 1;
    while (sub < 8 && blocks * sub * 2 <= (i64)cu_count() && tiles >= 4 * splits * sub * 2 && !empty_split(SK, splits * sub * 2))
        sub *= 2;
    return sub;
}

}  // namespace

extern "C" {

int fmha_mxfp8_kv_partials(int64_t B, int64_t H, int64_t S, int64_t SK, int splits) {
    if (B < 1 || H < 1 || S < 1 || SK < 1 || splits < 1) return 0;
    return (int)(splits * kv_fill(B, H, S, SK, splits));
}

const char* fmha_mxfp8_version(void) { return "fmha_mxfp8 gfx950 1.0"; }

int fmha_mxfp8_init(char* err, size_t errlen) {
    hipFunction_t* fns = nullptr;
    return get_functions(&fns, err, errlen);
}

int fmha_mxfp8_validate_vs128(const fmha_mxfp8_args* a, const fmha_mxfp8_buffer_sizes* sz, uint32_t gx, uint32_t gy,
                              uint32_t gz, int64_t HK, char* err, size_t errlen) {
    // the causal q-tile pairing runs on the 128-row grid only
    if (a->flags & FMHA_FLAG_CAUSAL_PAIR) return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "ka(0x280) outside contract");
    return validate_base(*a, *sz, gx, gy, (i64)gz, HK, 256, err, errlen);
}

int fmha_mxfp8_validate_t128(const fmha_mxfp8_args* a, const fmha_mxfp8_buffer_sizes* sz, uint32_t gx, uint32_t gy,
                             uint32_t gz, int64_t HK, char* err, size_t errlen) {
    return validate_base(*a, *sz, gx, gy, (i64)gz, HK, 128, err, errlen);
}

int fmha_mxfp8_validate_kvsplit(const fmha_mxfp8_kvsplit_args* ka, const fmha_mxfp8_buffer_sizes* sz, uint32_t gx,
                                uint32_t gy, uint32_t gz, int64_t B, int64_t HK, int64_t KL, char* err, size_t errlen) {
    // kvsplit_abi.h: the base rules with the symbol B, the split extension inserted into each group
    fmha_mxfp8_args a;
    std::memcpy(&a, ka, 0x270);
    std::memset(reinterpret_cast<uint8_t*>(&a) + 0x270, 0, sizeof(a) - 0x270);
    // the split count is the low 16 bits; bit 16 is the f32-partials extension (FMHA_KVS_F32_PARTIALS)
    const i64 splits = ka->kvs_splits & 0xffffu, rows = ka->kvs_rows_total;
    const i64 row_bytes = 512;   // the workspace rows are fp32-sized in both formats
    int rc;
    if ((rc = rules_extent(a, *sz, B, (ka->kvs_splits & FMHA_KVS_V_SEQ32) != 0, err, errlen)) != FMHA_OK) return rc;
    if (sz->ptr_ohat < (uint64_t)(splits * rows * row_bytes)) return fail(err, errlen, FMHA_ERR_EXTENT, "GV-HOST-EXTENT", "ptr_ohat: buffer ptr_ohat smaller than declared allocation");
    if (splits * rows * row_bytes >= (1LL << 32)) return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "ka(0x284) outside contract (partials of 4 GiB or more)");
    if (sz->ptr_lse < (uint64_t)(splits * rows * 4)) return fail(err, errlen, FMHA_ERR_EXTENT, "GV-HOST-EXTENT", "ptr_lse: buffer ptr_lse smaller than declared allocation");
    if ((rc = rules_range(a, err, errlen)) != FMHA_OK) return rc;
    if (splits < 1 || (ka->kvs_splits & ~(0xffffu | FMHA_KVS_F32_PARTIALS | FMHA_KVS_V_SEQ32 | FMHA_KVS_SCALE)) != 0)
        return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "ka(0x280) outside contract");
    if ((rc = rules_scale(a, (ka->kvs_splits & FMHA_KVS_SCALE) != 0, err, errlen)) != FMHA_OK) return rc;
    if (rows < 1) return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "ka(0x284) outside contract");
    if ((rc = rules_is(a, HK, err, errlen)) != FMHA_OK) return rc;
    if (rows != B * (i64)a.s_seq_len * (i64)a.s_q_head_num) return fail(err, errlen, FMHA_ERR_KA_IS, "GV-HOST-KA-IS", "ka(0x284) relation failed");
    if ((rc = rules_grid(a, gx, gy, 256, err, errlen)) != FMHA_OK) return rc;
    if ((i64)gz != B * splits) return fail(err, errlen, FMHA_ERR_GRID, "GV-HOST-GRID", "grid axis 2 relation failed");
    if (KL < 0) return fail(err, errlen, FMHA_ERR_SYM, "GV-HOST-SYM", "symbol KL outside contract");
    return FMHA_OK;
}

int fmha_mxfp8_validate_combine(const fmha_mxfp8_combine_args* a, const fmha_mxfp8_buffer_sizes* sz, uint32_t gx,
                                uint32_t gy, uint32_t gz, char* err, size_t errlen) {
    // combine8h_abi.h:56-65
    (void)gx; (void)gy; (void)gz;
    const i64 rows = a->rows_total, splits = a->splits & 0xffffu;
    if (sz->ptr_ohat < (uint64_t)(splits * rows * 512)) return fail(err, errlen, FMHA_ERR_EXTENT, "GV-HOST-EXTENT", "ptr_ohat: buffer ptr_ohat smaller than declared allocation");
    if (sz->ptr_lse < (uint64_t)(splits * rows * 4)) return fail(err, errlen, FMHA_ERR_EXTENT, "GV-HOST-EXTENT", "ptr_lse: buffer ptr_lse smaller than declared allocation");
    if (splits * rows * 512 >= (1LL << 32)) return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "ka(0x18) outside contract (partials of 4 GiB or more)");
    if (sz->ptr_o < (uint64_t)(rows * 256)) return fail(err, errlen, FMHA_ERR_EXTENT, "GV-HOST-EXTENT", "ptr_out: buffer ptr_out smaller than declared allocation");
    if (rows < 1) return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "ka(0x18) outside contract");
    if (a->d != 128) return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "ka(0x1C) outside contract");
    if (splits < 1 || (a->splits & ~(0xffffu | FMHA_KVS_F32_PARTIALS)) != 0)
        return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "ka(0x20) outside contract");
    return FMHA_OK;
}

int fmha_mxfp8_uses_split_tiles(int path, int64_t B, int64_t H, int64_t S, int64_t SK, int causal) {
    if (path == FMHA_PATH_T128) return use_split_tiles(B, H, S, SK, causal != 0) ? 1 : 0;
    if (path == FMHA_PATH_VS128)
        return vs128_on_128row_grid(B, H, S, SK, causal != 0) && use_split_tiles(B, H, S, SK, causal != 0) ? 1 : 0;
    return 0;
}

int fmha_mxfp8_select_path(int64_t B, int64_t H, int64_t S, int64_t SK, int* splits) {
    // dispatch.rs:494-511
    const i64 blocks256 = (S + 255) / 256 * H * B;
    const i64 ntiles = (SK + 127) / 128;
    i64 sp = 0;
    if (ntiles >= 16 && blocks256 <= 64) sp = 4;
    else if (ntiles >= 32 && blocks256 <= 128) sp = 2;
    if (sp > 0 && !empty_split(SK, sp)) {
        if (splits) *splits = (int)sp;
        return FMHA_PATH_KVSPLIT;
    }
    if (splits) *splits = 0;
    return blocks256 <= 64 ? FMHA_PATH_T128 : FMHA_PATH_VS128;
}

void fmha_mxfp8_fill_args(fmha_mxfp8_args* a, void* o, const void* q, const void* k, const void* v, const void* q_descale,
                          const void* k_descale, const void* v_descale, int B, int H, int HK, int S, int SK) {
    // the values tests/gpu/ref_host.cpp:342-360 writes
    (void)B;
    std::memset(a, 0, sizeof(*a));
    const uint32_t D = 128;
    a->ptr_o = o;
    a->ptr_q = const_cast<void*>(q);
    a->ptr_k = const_cast<void*>(k);
    a->ptr_v = const_cast<void*>(v);
    a->s_seq_len = (uint32_t)S;
    a->s_Seqs = (uint32_t)H * D;
    a->s_Hs = D;
    a->s_Bs = (uint32_t)((uint64_t)S * H * D);
    a->s_gqa = (uint32_t)(H / HK);
    a->s_k_Seqs = (uint32_t)HK * D;
    a->s_k_Hs = D;
    a->s_k_Bs = (uint32_t)((uint64_t)SK * HK * D);
    a->s_kv_seq_len = (uint32_t)SK;
    a->s_q_head_num = (uint32_t)H;
    a->s_v_Seqs = (uint32_t)HK * D;
    a->s_v_Hs = D;
    a->s_v_Bs = (uint32_t)((uint64_t)SK * HK * D);
    a->s_o_Seqs = (uint32_t)H * D * 2;
    a->s_o_Hs = D * 2;
    a->s_o_Bs = (uint32_t)((uint64_t)S * H * D * 2);
    a->ptr_q_descale = const_cast<void*>(q_descale);
    a->ptr_k_descale = const_cast<void*>(k_descale);
    a->ptr_v_descale = const_cast<void*>(v_descale);
    a->s_descale_q_Bs = (uint32_t)((uint64_t)S * H * 4);
    a->s_descale_q_Hs = 4;
    a->s_descale_k_Bs = (uint32_t)((uint64_t)SK * HK * 4);
    a->s_descale_k_Hs = 4;
    const float scale = 0.08838834764831845f;   // 1/sqrt(128), written as the reference host does (ignored)
    std::memcpy(&a->softmax_scale, &scale, 4);
}

size_t fmha_mxfp8_workspace_bytes(int64_t B, int64_t H, int64_t S, int splits) {
    if (splits <= 0) return 0;
    const uint64_t rows = (uint64_t)B * (uint64_t)S * (uint64_t)H;
    return (size_t)((uint64_t)splits * rows * (512u + 4u));
}

int fmha_mxfp8_launch_vs128(const fmha_mxfp8_args* a, uint32_t gx, uint32_t gy, uint32_t gz, void* stream) {
    return launch_raw((a->flags & FMHA_FLAG_SCALE) ? K_VS128_SC : K_VS128, a, sizeof(*a), gx, gy, gz, 512, stream, nullptr, 0);
}
int fmha_mxfp8_launch_t128(const fmha_mxfp8_args* a, uint32_t gx, uint32_t gy, uint32_t gz, void* stream) {
    // the reference-named kernel under its own contract: 256 threads (t128_abi.h)
    return launch_raw((a->flags & FMHA_FLAG_SCALE) ? K_T128_SC : K_T128, a, sizeof(*a), gx, gy, gz, 256, stream, nullptr, 0);
}
int fmha_mxfp8_launch_t128_split_tiles(const fmha_mxfp8_args* a, uint32_t gx, uint32_t gy, uint32_t gz, void* stream) {
    return launch_raw((a->flags & FMHA_FLAG_SCALE) ? K_T128ST_SC : K_T128ST, a, sizeof(*a), gx, gy, gz, 512, stream, nullptr, 0);
}
int fmha_mxfp8_launch_kvsplit(const fmha_mxfp8_kvsplit_args* a, uint32_t gx, uint32_t gy, uint32_t gz, void* stream) {
    return launch_raw((a->kvs_splits & FMHA_KVS_SCALE) ? K_KVSPLIT_SC : K_KVSPLIT, a, sizeof(*a), gx, gy, gz, 512, stream, nullptr, 0);
}
int fmha_mxfp8_launch_combine(const fmha_mxfp8_combine_args* a, uint32_t gx, void* stream) {
    return launch_raw(K_COMBINE, a, sizeof(*a), gx, 1, 1, 256, stream, nullptr, 0);
}
int fmha_mxfp8_launch_combine_wide(const fmha_mxfp8_combine_args* a, uint32_t gx, void* stream) {
    return launch_raw(K_COMBINE_WIDE, a, sizeof(*a), gx, 1, 1, 256, stream, nullptr, 0);
}

int fmha_fwd_hd128_mxfp8_auto(const fmha_mxfp8_params* p, void* workspace, size_t workspace_bytes, void* stream, int* path_out,
                              int* splits_out, char* err, size_t errlen) {
    if (!p) return fail(err, errlen, FMHA_ERR_PATH, "GV-HOST-ARGS", "null params");
    const i64 B = p->B, H = p->H, HK = p->HK, S = p->S, SK = p->SK;
    if (B < 1 || H < 1 || HK < 1 || S < 1 || SK < 1)
        return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "B, H, HK, S, SK must be >= 1");
    if (H % HK != 0 || ((H / HK) & (H / HK - 1)) != 0 || H / HK > 16)
        return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "H must be a power-of-two multiple (<= 16) of HK");
    int splits = 0;
    int path = p->path;
    if (path < 0) {
        path = fmha_mxfp8_select_path(B, H, S, SK, &splits);
        if (p->causal && path == FMHA_PATH_KVSPLIT) path = ((S + 255) / 256 * H * B <= 64) ? FMHA_PATH_T128 : FMHA_PATH_VS128;
    } else if (path == FMHA_PATH_KVSPLIT) {
        splits = p->splits > 0 ? p->splits : 4;
    }
    if (path != FMHA_PATH_VS128 && path != FMHA_PATH_T128 && path != FMHA_PATH_KVSPLIT)
        return fail(err, errlen, FMHA_ERR_PATH, "GV-HOST-PATH", "unknown path");
    if (path == FMHA_PATH_KVSPLIT) {
        if (splits != 2 && splits != 4 && splits != 8) return fail(err, errlen, FMHA_ERR_PATH, "GV-HOST-PATH", "KV split count must be 2, 4 or 8");
        if (empty_split(SK, splits)) return fail(err, errlen, FMHA_ERR_PATH, "GV-HOST-PATH", "KV split leaves a split without a key tile");
        if (p->causal) return fail(err, errlen, FMHA_ERR_PATH, "GV-HOST-PATH", "the causal mask is not supported on the KV-split path");
    }
    if (p->f32_partials != 0 && p->f32_partials != 1)
        return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "f32_partials must be 0 or 1");
    if (p->v_seq32 != 0 && p->v_seq32 != 1)
        return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "v_seq32 must be 0 or 1");
    if (p->causal_pair < 0 || p->causal_pair > 2)
        return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "causal_pair must be 0, 1 or 2");
    if (p->kv_fill != 0 && p->kv_fill != 1)
        return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "kv_fill must be 0 or 1");
    const bool scaled = p->softmax_scale != 0.0f;
    if (scaled && !scale_ok(p->softmax_scale))
        return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "softmax_scale must be 0 or positive with a normal f32 scale x log2(e)");
    fmha_mxfp8_args a;
    fmha_mxfp8_fill_args(&a, p->o, p->q, p->k, p->v, p->q_descale, p->k_descale, p->v_descale, (int)B, (int)H, (int)HK, (int)S, (int)SK);
    a.flags = (p->causal ? FMHA_FLAG_CAUSAL : 0u) | (p->v_seq32 ? FMHA_FLAG_V_SEQ32 : 0u) | (scaled ? FMHA_FLAG_SCALE : 0u);
    if (scaled) std::memcpy(&a.softmax_scale, &p->softmax_scale, 4);
    fmha_mxfp8_buffer_sizes sz;
    std::memset(&sz, 0, sizeof(sz));
    sz.ptr_q = p->bytes_q; sz.ptr_k = p->bytes_k; sz.ptr_v = p->bytes_v; sz.ptr_o = p->bytes_o;
    sz.ptr_q_descale = p->bytes_q_descale; sz.ptr_k_descale = p->bytes_k_descale; sz.ptr_v_descale = p->bytes_v_descale;
    // the KV split's partial count: the chunks times the fill, as far as the workspace holds it
    i64 parts = splits;
    if (path == FMHA_PATH_KVSPLIT) {
        i64 sub = p->kv_fill ? 1 : kv_fill(B, H, S, SK, splits);
        while (sub > 1 && workspace_bytes < fmha_mxfp8_workspace_bytes(B, H, S, (int)(splits * sub))) sub /= 2;
        parts = splits * sub;
    }
    if (path == FMHA_PATH_KVSPLIT && parts * B * S * H * 512 >= (1LL << 32))
        // a kernel-contract limit (32-bit partial offsets), checked with or without no_check
        return fail(err, errlen, FMHA_ERR_KA_RANGE, "GV-HOST-KA-RANGE", "ka(0x284) outside contract (partials of 4 GiB or more)");
    if (path_out) *path_out = path;
    if (splits_out) *splits_out = path == FMHA_PATH_KVSPLIT ? splits : 0;
    if (p->partials_out) *p->partials_out = path == FMHA_PATH_KVSPLIT ? (int32_t)parts : 0;
    const uint32_t gy = (uint32_t)H;
    if (path == FMHA_PATH_VS128 || path == FMHA_PATH_T128) {
        a.ptr_lse = p->lse;
        const int rows = path == FMHA_PATH_VS128 ? 256 : 128;
        const uint32_t gx = (uint32_t)((S + rows - 1) / rows);
        if (!p->no_check) {
            const int rc = path == FMHA_PATH_VS128 ? fmha_mxfp8_validate_vs128(&a, &sz, gx, gy, (uint32_t)B, HK, err, errlen)
                                                   : fmha_mxfp8_validate_t128(&a, &sz, gx, gy, (uint32_t)B, HK, err, errlen);
            if (rc != FMHA_OK) return rc;
        }
        uint32_t block = 512u, kgx = gx;
        int kern;
        if (path == FMHA_PATH_VS128 && !vs128_on_128row_grid(B, H, S, SK, p->causal != 0)) {
            kern = scaled ? K_VS128_SC : K_VS128;
        } else {
            // t128, or vs128 on the 128-row grid (same kernarg layout): the split-tile kernel or the 256-thread one
            const bool st = use_split_tiles(B, H, S, SK, p->causal != 0);
            kern = st ? (scaled ? K_T128ST_SC : K_T128ST) : (scaled ? K_T128_SC : K_T128);
            block = st ? 512u : 256u;
            kgx = (uint32_t)((S + 127) / 128);
        }
        // the causal q-tile pairing when the grid would take more than one wave of blocks (the extension's flag; the
        // reference pairs its causal kernels' tiles always, grid.rs:94-111), or when the caller asks for it
        const bool pair = p->causal && kern != K_VS128 && kern != K_VS128_SC && kgx > 1 &&
                          (p->causal_pair == 1 || (p->causal_pair == 0 && (i64)kgx * H * B > (i64)cu_count()));
        if (pair) {
            a.flags |= FMHA_FLAG_CAUSAL_PAIR;
            kgx = (kgx + 1) / 2;
        }
        return launch_raw(kern, &a, sizeof(a), kgx, gy, (uint32_t)B, block, stream, err, errlen);
    }
    // KV split: partials (fp32-sized rows, as ref_host.cpp:149 / ops.py:133) then the LSE, both in the workspace
    const i64 rows_total = B * S * H;
    const size_t need = fmha_mxfp8_workspace_bytes(B, H, S, (int)parts);
    if (!workspace || workspace_bytes < need) {
        set_err(err, errlen, "GV-HOST-WORKSPACE: KV split needs %zu workspace bytes, got %zu", need, workspace_bytes);
        return FMHA_ERR_WORKSPACE;
    }
    // Workspace slots: a workspace of k >= 2 times the need (rounded to 256 B) holds min(k, FMHA_WORKSPACE_SLOTS) sets
    // of partials, and consecutive calls take them in turn. The split kernel then writes lines that the previous
    // call's combine did not just read: writing over partials that the combine read in the kernel before cost
    // B1H8S2048 (4 splits) 25.6 -> 19.1 us per call with 4 slots (2 slots: 21.2, 8: 19.1, 16: 20.0).
    const size_t stride = (need + 255u) & ~(size_t)255u;
    size_t nslots = workspace_bytes / stride;
    if (nslots < 1) nslots = 1;
    if (nslots > FMHA_WORKSPACE_SLOTS) nslots = FMHA_WORKSPACE_SLOTS;
    size_t slot = 0;
    if (nslots > 1 && p->ws_turn) slot = (size_t)((*p->ws_turn)++ % nslots);
    uint8_t* ohat = (uint8_t*)workspace + slot * stride;
    uint8_t* lse = ohat + (size_t)parts * rows_total * 512;
    fmha_mxfp8_kvsplit_args ka;
    std::memcpy(&ka, &a, 0x270);
    ka.ptr_ohat = ohat;
    ka.ptr_lse = lse;
    const uint32_t part_fmt = p->f32_partials ? FMHA_KVS_F32_PARTIALS : 0u;
    ka.kvs_splits = (uint32_t)parts | part_fmt | (p->v_seq32 ? FMHA_KVS_V_SEQ32 : 0u) | (scaled ? FMHA_KVS_SCALE : 0u);
    ka.kvs_rows_total = (uint32_t)rows_total;
    sz.ptr_ohat = (uint64_t)parts * rows_total * 512;
    sz.ptr_lse = (uint64_t)parts * rows_total * 4;
    const uint32_t gx = (uint32_t)((S + 255) / 256), gz = (uint32_t)(B * parts);
    int rc = p->no_check ? FMHA_OK : fmha_mxfp8_validate_kvsplit(&ka, &sz, gx, gy, gz, B, HK, 0, err, errlen);
    if (rc != FMHA_OK) return rc;
    rc = launch_raw(scaled ? K_KVSPLIT_SC : K_KVSPLIT, &ka, sizeof(ka), gx, gy, gz, 512, stream, err, errlen);
    if (rc != FMHA_OK) return rc;
    fmha_mxfp8_combine_args ca;
    ca.ptr_ohat = ohat;
    ca.ptr_lse = lse;
    ca.ptr_out = p->o;
    ca.rows_total = (uint32_t)rows_total;
    ca.d = 128;
    ca.splits = (uint32_t)parts | part_fmt;
    fmha_mxfp8_buffer_sizes csz = sz;
    csz.ptr_o = p->bytes_o;
    if (!p->no_check) {
        rc = fmha_mxfp8_validate_combine(&ca, &csz, 0, 1, 1, err, errlen);
        if (rc != FMHA_OK) return rc;
    }
    // more than 8 partials per row: the combine with the splits spread over 4 waves (64 groups per block)
    const bool wide = parts > 8;
    const uint64_t cgrid = ((uint64_t)rows_total * 128 / 8 + (wide ? 63 : 255)) / (wide ? 64 : 256);
    return launch_raw(wide ? K_COMBINE_WIDE : K_COMBINE, &ca, sizeof(ca), (uint32_t)(cgrid ? cgrid : 1), 1, 1, 256, stream, err,
                      errlen);
}

}  // extern "C"
