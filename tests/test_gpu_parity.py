"""GPU parity of the HIP kernels against the CPU oracle (oracle/), through the C ABI.

Parity bar: per shape, mean |err| against the fp64 attention on the dequantised
inputs <= 1.10 x the reference kernel's and bad count (|err| > 0.05 + 0.05 |ref|) <= the reference's, both on
the first 64 query rows of every (b, h) (tests/gpu/ref_host.cpp:436-471). "The reference kernel's" error is the
bit-level emulation of its recipe (oracle.emulate), which reproduces the reference's published per-shape
statistics (tests/test_oracle.py). Beyond the bar, the output must stay close to that emulation element-wise.
It cannot be bit-identical: the gfx950 scaled fp8 MFMA does not sum its 64 products exactly (measured: errors up to
~3e-4 of the largest product), which moves the fp8 rounding of some P values; the emulation sums exactly. The
element-wise bound therefore is a fraction of the reference's own error, not zero.
"""
import ctypes

import numpy as np
import pytest

import oracle
from amdgpu_rustdsl_amd import lib, ops
from tests import gpu_util

pytestmark = pytest.mark.gpu

ROWS = 64

# (name, B, H, HK, S, SK, causal, path, splits)
CASES = [
    ("cfg1_B1H1S256", 1, 1, 1, 256, 256, False, "auto", None),
    ("cfg2_B4H8S2048", 4, 8, 8, 2048, 2048, False, "auto", None),
    ("cfg3_B1H8S8192", 1, 8, 8, 8192, 8192, False, "auto", None),
    ("cfg5_B1H8S128_SK16384_split8", 1, 8, 8, 128, 16384, False, "kvsplit", 8),
    ("cfg5_B1H8S128_SK16000_split8", 1, 8, 8, 128, 16000, False, "kvsplit", 8),
    ("auto_split4_B1H8S2048", 1, 8, 8, 2048, 2048, False, "auto", None),
    ("t128_ragged_B1H8S1000_SK1337", 1, 8, 8, 1000, 1337, False, "auto", None),
    ("vs128_ragged_B2H8S2100_SK333", 2, 8, 8, 2100, 333, False, "vs128", None),
    ("gqa4_B1H8HK2_S2048", 1, 8, 2, 2048, 2048, False, "kvsplit", 4),
    ("gqa2_vs128_B4H8HK4_S1024", 4, 8, 4, 1024, 1024, False, "vs128", None),
    ("tiny_S1_SK1", 1, 2, 2, 1, 1, False, "auto", None),
    ("short_SK129", 1, 4, 4, 300, 129, False, "auto", None),
    ("split2_SK4096", 1, 4, 4, 512, 4096, False, "kvsplit", 2),
]


def _emulated_bar(inp, splits, rows=ROWS, path=None, ref_splits=None, **kw):
    """The reference's error statistics (its order, on its `ref_splits` KV chunks, default `splits`), and the
    emulation to compare element-wise with: the library's own order on the `splits` partials that ran (the chunks
    times the blocks each was spread over), which also differs from the reference's for KV-split blocks of at most
    128 query rows and where the one-call entry runs a full-sequence path on the split-tile kernel
    (lib.uses_split_tiles; not with the LUT recipe, which the emulation handles)."""
    ref_splits = splits if ref_splits is None else ref_splits
    emu = oracle.emulate(inp, splits=ref_splits, rows=rows, **kw)
    ref_stats = oracle.check_fp64(inp, emu, rows=rows)
    if splits or (path is not None and lib.uses_split_tiles(path, inp.B, inp.H, inp.S, inp.SK, inp.causal)):
        emu = oracle.emulate(inp, splits=splits, rows=rows, split_tiles=True, **kw)
    return emu, ref_stats


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_parity(gpu, case):
    name, B, H, HK, S, SK, causal, path, splits = case
    print(f"[case] {name}", flush=True)
    inp = oracle.Inputs(B, H, S, SK, HK=HK, causal=causal)
    out, used, _ = gpu_util.run(inp, gpu, path=path, splits=splits)
    used_splits = used.partials if used[0] == "kvsplit" else 0
    # the reference's sample (the first 64 rows of every (b, h)) and the last 64: the last query tile and the tail
    rows = oracle.first_and_last(S, ROWS)
    emu, ref_stats = _emulated_bar(inp, used_splits, rows=rows, path=used[0], ref_splits=gpu_util.chunks(inp, path, splits))
    stats = oracle.check_fp64(inp, out, rows=rows)
    cmp = gpu_util.compare_to_emulation(out, emu, inp, rows)
    print(f"[case] {name} path={used} ours={stats} emulated-reference={ref_stats} vs-emulation={cmp}", flush=True)
    # every element written (the output was NaN-poisoned), full tensor
    assert not np.isnan(oracle.bf16_to_f32(out)).any(), "unwritten / NaN outputs"
    assert stats["bad"] <= ref_stats["bad"]
    assert stats["mean_err"] <= 1.10 * ref_stats["mean_err"]
    # same recipe: element-wise closeness to the emulation (MFMA-internal summation differences only)
    assert cmp["mean_abs"] <= 0.6 * ref_stats["mean_err"], cmp
    assert cmp["max_abs"] <= 0.05, cmp


# Extensions (no counterpart in the reference kernels): the bottom-right causal mask and the LSE output. Their bar is
# the same statistical one against the oracle's emulation of the recipe with the mask applied (oracle.emulate honours
# Inputs.causal; its mask is pinned against numpy in tests/test_oracle.py).
CAUSAL_CASES = [
    ("causal_cfg4_B2H8S2048", 2, 8, 8, 2048, 2048),
    ("causal_ragged_B1H4S1000_SK1337", 1, 4, 4, 1000, 1337),
    ("causal_S_gt_SK_B1H2S700_SK300", 1, 2, 2, 700, 300),   # rows with no visible key produce zeros
    ("causal_t128_B1H2S512", 1, 2, 2, 512, 512),
]


@pytest.mark.parametrize("case", CAUSAL_CASES, ids=[c[0] for c in CAUSAL_CASES])
def test_parity_causal(gpu, case):
    name, B, H, HK, S, SK = case
    print(f"[case] {name}", flush=True)
    inp = oracle.Inputs(B, H, S, SK, HK=HK, causal=True)
    out, used, _ = gpu_util.run(inp, gpu)
    assert used[0] in ("vs128", "t128")
    # rows checked: all of them for the small shapes; for cfg4 the first 128 of every (b, h) (the mask cuts every
    # tile they see) and the last 128 (they see all 16 key tiles: the many-tile lazy rebase under the mask)
    rows = S if B * H * S * SK <= (1 << 24) else oracle.first_and_last(S, 128)
    emu, ref_stats = _emulated_bar(inp, 0, rows=rows, path=used[0])
    stats = oracle.check_fp64(inp, out, rows=rows)
    cmp = gpu_util.compare_to_emulation(out, emu, inp, rows)
    fig, viol = gpu_util.causal_bar(inp, out, emu, rows)
    print(f"[case] {name} path={used} ours={stats} emulated-reference={ref_stats} vs-emulation={cmp} causal-bar={fig}", flush=True)
    assert not np.isnan(oracle.bf16_to_f32(out)).any()
    assert stats["bad"] <= ref_stats["bad"]
    assert stats["mean_err"] <= 1.10 * ref_stats["mean_err"] + 1e-7
    assert cmp["mean_abs"] <= 0.6 * max(ref_stats["mean_err"], 1e-6), cmp
    assert not viol, (viol, fig)   # per-row element bound by visible-key count (gpu_util.causal_bar)
    if S > SK:
        o = oracle.bf16_to_f32(out).reshape(B, S, H, 128)
        assert (o[:, : S - SK] == 0).all()   # query i sees keys t <= i + SK - S: none for i < S - SK


# Extension: the KV split with f32 partial rows (partials="fp32"; the reference writes fp16). Bar: the statistical one
# against the oracle's emulation of the same variant, and no worse than the fp16 variant of the GPU path itself.
F32_CASES = [
    ("cfg5_B1H8S128_SK16384_split8", 1, 8, 8, 128, 16384, 8),
    ("cfg5_B1H8S128_SK16000_split8", 1, 8, 8, 128, 16000, 8),
    ("gqa4_B1H8HK2_S2048_split4", 1, 8, 2, 2048, 2048, 4),
    ("split2_B1H4S300_SK1000", 1, 4, 4, 300, 1000, 2),
]


@pytest.mark.parametrize("case", F32_CASES, ids=[c[0] for c in F32_CASES])
def test_parity_f32_partials(gpu, case):
    name, B, H, HK, S, SK, splits = case
    print(f"[case] f32 partials {name}", flush=True)
    inp = oracle.Inputs(B, H, S, SK, HK=HK)
    out, used, _ = gpu_util.run(inp, gpu, path="kvsplit", splits=splits, partials="fp32")
    assert used == ("kvsplit", splits) and used.partials == lib.kv_partials(B, H, S, SK, splits)
    out16, _, _ = gpu_util.run(inp, gpu, path="kvsplit", splits=splits)
    emu, ref_stats = _emulated_bar(inp, used.partials, f32_partials=True, ref_splits=splits)
    stats = oracle.check_fp64(inp, out, rows=ROWS)
    stats16 = oracle.check_fp64(inp, out16, rows=ROWS)
    cmp = gpu_util.compare_to_emulation(out, emu, inp, min(ROWS, S))
    print(f"[case] f32 partials {name} ours={stats} fp16-partials={stats16} emulated={ref_stats} vs-emulation={cmp}", flush=True)
    assert not np.isnan(oracle.bf16_to_f32(out)).any()
    assert stats["bad"] <= ref_stats["bad"]
    assert stats["mean_err"] <= 1.10 * ref_stats["mean_err"]
    assert stats["mean_err"] <= stats16["mean_err"] * 1.01
    assert cmp["mean_abs"] <= 0.6 * ref_stats["mean_err"], cmp
    assert cmp["max_abs"] <= 0.05, cmp


# Extension: per-32-key V scales (V re-quantised with one E8M0 per 32 keys per column; the PV MFMAs apply them).
# Bar: the statistical one against the oracle's emulation of the same inputs, and element-wise closeness to it.
VS32_CASES = [
    ("vs128_B2H8S1024", 2, 8, 8, 1024, 1024, False, "vs128", None),
    ("vs128_ragged_B1H8HK2_S700_SK1000", 1, 8, 2, 700, 1000, False, "vs128", None),   # SK % 32 != 0, GQA 4
    ("t128_B1H4S512_SK600", 1, 4, 4, 512, 600, False, "t128", None),
    ("t128_short_SK100", 1, 2, 2, 256, 100, False, "t128", None),                     # < 4 tiles: the LUT recipe
    ("kvsplit_B1H8S128_SK4000_split4", 1, 8, 8, 128, 4000, False, "kvsplit", 4),
    ("causal_vs128_B1H8S1024", 1, 8, 8, 1024, 1024, True, "vs128", None),
]


@pytest.mark.parametrize("case", VS32_CASES, ids=[c[0] for c in VS32_CASES])
def test_parity_v_seq32(gpu, case):
    name, B, H, HK, S, SK, causal, path, splits = case
    print(f"[case] v_seq32 {name}", flush=True)
    inp = oracle.Inputs(B, H, S, SK, HK=HK, causal=causal, v_seq32=True)
    out, used, _ = gpu_util.run(inp, gpu, path=path, splits=splits)
    assert used[0] == path
    used_splits = used.partials if used[0] == "kvsplit" else 0
    rows = oracle.first_and_last(S, 128 if causal else ROWS)
    emu, ref_stats = _emulated_bar(inp, used_splits, rows=rows, path=used[0], ref_splits=gpu_util.chunks(inp, path, splits))
    stats = oracle.check_fp64(inp, out, rows=rows)
    cmp = gpu_util.compare_to_emulation(out, emu, inp, rows)
    print(f"[case] v_seq32 {name} path={used} ours={stats} emulated={ref_stats} vs-emulation={cmp}", flush=True)
    assert not np.isnan(oracle.bf16_to_f32(out)).any()
    assert stats["bad"] <= ref_stats["bad"]
    assert stats["mean_err"] <= 1.10 * ref_stats["mean_err"]
    assert cmp["mean_abs"] <= 0.6 * ref_stats["mean_err"], cmp
    assert cmp["max_abs"] <= 0.05, cmp


@pytest.mark.parametrize("scale", [0.0, 0.7], ids=["", "scale0.7"])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("shape", [(1, 4, 4, 512, 640), (4, 8, 8, 1024, 1024), (4, 8, 8, 2048, 2048)],
                         ids=["t128", "vs128_split_tiles", "vs128"])
def test_lse_output(gpu, shape, causal, scale):
    """The optional natural-log LSE (kernarg 0x040): log sum_t exp(ln2 c q.k_t) over the visible keys, against
    float64 (c = 1, or the in-kernel softmax scale's multiplier)."""
    B, H, HK, S, SK = shape
    inp = oracle.Inputs(B, H, S, SK, HK=HK, causal=causal, qk_scale=scale)
    out, used, lse_t = gpu_util.run(inp, gpu, lse=True)
    lse = lse_t.cpu().numpy()
    # under the mask every row: the first 64 see 1..64 keys, so the rows that see many keys come from further down
    nrow = S if causal else 64
    ref = gpu_util.lse_reference(inp, rows=nrow)
    got = lse[:, :, :nrow]
    err = np.abs(got - ref)
    print(f"[case] lse {shape} causal={causal} scale={scale} path={used} max_err={err.max():.3g} mean_err={err.mean():.3g}",
          flush=True)
    assert np.isfinite(got).all()
    assert used[0] == ("t128" if S == 512 else "vs128")
    # l sums the recipe's P: an exp2 approximation (per key within a factor 1.087 of 2^x, bias removed on average) then
    # e4m3 rounding. A row with few visible keys (causal, top rows) keeps its keys' approximation error, up to
    # ln 1.087 = 0.083; over many keys it averages out to a few 1e-3.
    assert err.max() < 0.09
    nvis = np.minimum(SK, np.arange(nrow) + SK - S + 1) if causal else np.full(nrow, SK)
    many = nvis >= 64
    assert err[:, :, many].mean() < 4e-3


# The KV split's split-tile order (blocks of at most 128 query rows: the two wave groups take keys 0..63 and 64..127
# of every tile and merge at the end), checked on every row, so that the ragged last block of S = 300 and the whole
# of S <= 128 are in: the bar is the reference's error statistics on those rows, and element-wise closeness to the
# oracle's emulation of the same order.
SPLIT_TILE_CASES = [
    ("S128_SK4096_split4", 1, 8, 8, 128, 4096, 4, {}),
    ("S300_SK2000_split2", 1, 4, 4, 300, 2000, 2, {}),                 # block 0: plain order, block 1 (44 rows): split
    ("S1_SK3000_split8", 2, 4, 4, 1, 3000, 8, {}),                      # one row; the last split's tile is ragged
    ("gqa4_S64_SK1000_split2", 1, 8, 2, 64, 1000, 2, {}),
    ("S128_SK1200_split4_f32", 1, 4, 4, 128, 1200, 4, {"partials": "fp32"}),
    ("S100_SK777_split2_vs32", 1, 4, 4, 100, 777, 2, {"v_seq32": True}),
]


@pytest.mark.parametrize("case", SPLIT_TILE_CASES, ids=[c[0] for c in SPLIT_TILE_CASES])
def test_parity_split_tiles(gpu, case):
    name, B, H, HK, S, SK, splits, opt = case
    print(f"[case] split tiles {name}", flush=True)
    inp = oracle.Inputs(B, H, S, SK, HK=HK, v_seq32=opt.get("v_seq32", False))
    f32 = opt.get("partials") == "fp32"
    out, used, _ = gpu_util.run(inp, gpu, path="kvsplit", splits=splits, partials=opt.get("partials", "fp16"))
    assert used == ("kvsplit", splits) and used.partials == lib.kv_partials(B, H, S, SK, splits)
    emu, ref_stats = _emulated_bar(inp, used.partials, rows=S, f32_partials=f32, ref_splits=splits)
    stats = oracle.check_fp64(inp, out, rows=S)
    cmp = gpu_util.compare_to_emulation(out, emu, inp, S)
    print(f"[case] split tiles {name} ours={stats} emulated-reference={ref_stats} vs-emulation={cmp}", flush=True)
    assert not np.isnan(oracle.bf16_to_f32(out)).any()
    assert stats["bad"] <= ref_stats["bad"]
    assert stats["mean_err"] <= 1.10 * ref_stats["mean_err"]
    assert cmp["mean_abs"] <= 0.6 * ref_stats["mean_err"], cmp
    assert cmp["max_abs"] <= 0.05, cmp


# Extension: the softmax scale applied in the kernel (kernarg 0x050 with FMHA_FLAG_SCALE / FMHA_KVS_SCALE): Q is the
# generator's, the scores become c q.k with c = f32(scale log2 e) = 2^e m, the exponent joining the Q scales and S
# multiplied by m. Bar: the statistical one against the oracle's emulation of the same arithmetic, on every path.
QK_SCALE_CASES = [
    ("vs128_B2H8S1024_c1", 2, 8, 8, 1024, 1024, False, False, "vs128", None, 0.6931471805599453),
    ("vs128_ragged_S700_SK1000_c2.16", 1, 8, 2, 700, 1000, False, False, "vs128", None, 1.5),
    ("t128_B1H4S512_SK600_c0.43", 1, 4, 4, 512, 600, False, False, "t128", None, 0.3),
    ("t128_lut_SK100_c1.44", 1, 2, 2, 256, 100, False, False, "t128", None, 1.0),
    ("kvsplit_S128_SK4096_split4_c0.72", 1, 8, 8, 128, 4096, False, False, "kvsplit", 4, 0.5),
    ("kvsplit_S300_SK2000_split2_c1.15", 1, 4, 4, 300, 2000, False, False, "kvsplit", 2, 0.8),
    ("causal_vs128_S1024_c1.3", 1, 8, 8, 1024, 1024, True, False, "vs128", None, 0.9),
    ("vs32_vs128_S512_SK777_c0.87", 1, 4, 4, 512, 777, False, True, "vs128", None, 0.6),
]


@pytest.mark.parametrize("case", QK_SCALE_CASES, ids=[c[0] for c in QK_SCALE_CASES])
def test_parity_qk_scale(gpu, case):
    name, B, H, HK, S, SK, causal, vs32, path, splits, scale = case
    print(f"[case] qk scale {name}", flush=True)
    inp = oracle.Inputs(B, H, S, SK, HK=HK, causal=causal, v_seq32=vs32, qk_scale=scale)
    out, used, _ = gpu_util.run(inp, gpu, path=path, splits=splits)
    assert used[0] == path
    used_splits = used.partials if used[0] == "kvsplit" else 0
    rows = S if path == "kvsplit" else oracle.first_and_last(S, 128 if causal else ROWS)
    emu, ref_stats = _emulated_bar(inp, used_splits, rows=rows, path=used[0], ref_splits=gpu_util.chunks(inp, path, splits))
    stats = oracle.check_fp64(inp, out, rows=rows)
    cmp = gpu_util.compare_to_emulation(out, emu, inp, rows)
    print(f"[case] qk scale {name} path={used} ours={stats} emulated={ref_stats} vs-emulation={cmp}", flush=True)
    assert not np.isnan(oracle.bf16_to_f32(out)).any()
    assert stats["bad"] <= ref_stats["bad"]
    assert stats["mean_err"] <= 1.10 * ref_stats["mean_err"] + 1e-7
    assert cmp["mean_abs"] <= 0.6 * max(ref_stats["mean_err"], 1e-6), cmp
    assert cmp["max_abs"] <= 0.05, cmp


# The t128 path's split-tile kernel (extension: 512 threads on t128's 128-row blocks, the two wave groups splitting each
# tile's keys), on every row: shapes of the reference's t128 dispatch, GQA, a ragged tail, causal, and through the
# direct launcher fmha_mxfp8_launch_t128_split_tiles.
T128_ST_CASES = [
    ("B1H8S1024", 1, 8, 8, 1024, 1024, False),
    ("B2H8S512_SK1024_gqa4", 2, 8, 2, 512, 1024, False),
    ("B1H8S1000_SK1337", 1, 8, 8, 1000, 1337, False),
    ("B1H4S700_SK700_causal", 1, 4, 4, 700, 700, True),
    ("B1H2S100_SK2000", 1, 2, 2, 100, 2000, False),
]


@pytest.mark.parametrize("case", T128_ST_CASES, ids=[c[0] for c in T128_ST_CASES])
def test_parity_t128_split_tiles(gpu, case):
    name, B, H, HK, S, SK, causal = case
    print(f"[case] t128 split tiles {name}", flush=True)
    inp = oracle.Inputs(B, H, S, SK, HK=HK, causal=causal)
    out, used, _ = gpu_util.run(inp, gpu, path="t128")
    assert used[0] == "t128"
    emu, ref_stats = _emulated_bar(inp, 0, rows=S, path="t128")
    stats = oracle.check_fp64(inp, out, rows=S)
    cmp = gpu_util.compare_to_emulation(out, emu, inp, S)
    print(f"[case] t128 split tiles {name} ours={stats} emulated-reference={ref_stats} vs-emulation={cmp}", flush=True)
    assert not np.isnan(oracle.bf16_to_f32(out)).any()
    assert stats["bad"] <= ref_stats["bad"]
    assert stats["mean_err"] <= 1.10 * ref_stats["mean_err"] + 1e-7
    assert cmp["mean_abs"] <= 0.6 * max(ref_stats["mean_err"], 1e-6), cmp
    assert cmp["max_abs"] <= 0.05, cmp
    if not causal:
        # the direct launcher of the same kernel (512 threads, t128's grid): bit-identical output
        import ctypes, math, torch
        from amdgpu_rustdsl_amd import lib
        q, k, v, qs, ks, vs = gpu_util.upload(inp, gpu)
        o2 = torch.full((B, S, H, 128), float("nan"), dtype=torch.bfloat16, device=gpu)
        a = lib.fill_args(o2.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), qs.data_ptr(), ks.data_ptr(), vs.data_ptr(),
                          B, H, HK, S, SK)
        st = torch.cuda.current_stream(gpu).cuda_stream
        assert lib.raw.fmha_mxfp8_launch_t128_split_tiles(ctypes.byref(a), math.ceil(S / 128), H, B, st) == 0
        torch.cuda.synchronize()
        direct = o2.view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)
        np.testing.assert_array_equal(direct, out)


# vs128 shapes whose 256-row grid holds at most 128 blocks: the one-call entry runs them on the split-tile kernel
# (t128's 128-row grid, 512 threads); (name, B, H, HK, S, SK, causal, path forced or None)
VS128_ST_CASES = [
    ("B2H8S2048", 2, 8, 8, 2048, 2048, False, None),
    ("B8H8S512_SK1024", 8, 8, 8, 512, 1024, False, None),
    ("B4H8HK2_S1024_gqa4", 4, 8, 2, 1024, 1024, False, None),
    ("B2H8S2048_SK1337", 2, 8, 8, 2048, 1337, False, None),
    ("B1H4S700_SK900_forced", 1, 4, 4, 700, 900, False, "vs128"),
    ("B2H4S1000_SK1000_causal_forced", 2, 4, 4, 1000, 1000, True, "vs128"),
]


@pytest.mark.parametrize("case", VS128_ST_CASES, ids=[c[0] for c in VS128_ST_CASES])
def test_parity_vs128_split_tiles(gpu, case):
    name, B, H, HK, S, SK, causal, force = case
    print(f"[case] vs128 split tiles {name}", flush=True)
    assert lib.uses_split_tiles("vs128", B, H, S, SK, causal)
    inp = oracle.Inputs(B, H, S, SK, HK=HK, causal=causal)
    out, used, _ = gpu_util.run(inp, gpu, path=force or "auto")
    assert used[0] == "vs128"
    # every row where the emulation is cheap (every q tile and its XCD-remapped block), else the first and the last q
    # tile of every (b, h)
    rows = S if B * H * S * SK <= 10_000_000 else oracle.first_and_last(S, 128)
    emu, ref_stats = _emulated_bar(inp, 0, rows=rows, path="vs128")
    stats = oracle.check_fp64(inp, out, rows=rows)
    cmp = gpu_util.compare_to_emulation(out, emu, inp, rows)
    print(f"[case] vs128 split tiles {name} ours={stats} emulated-reference={ref_stats} vs-emulation={cmp}", flush=True)
    assert not np.isnan(oracle.bf16_to_f32(out)).any()
    assert stats["bad"] <= ref_stats["bad"]
    assert stats["mean_err"] <= 1.10 * ref_stats["mean_err"] + 1e-7
    assert cmp["mean_abs"] <= 0.6 * max(ref_stats["mean_err"], 1e-6), cmp
    if causal:
        # under the mask the per-row element bound of test_parity_causal (gpu_util.causal_bar)
        fig, viol = gpu_util.causal_bar(inp, out, emu, rows)
        print(f"[case] vs128 split tiles {name} causal-bar={fig}", flush=True)
        assert not viol, (viol, fig)
    else:
        assert cmp["max_abs"] <= 0.05, cmp
    if not causal:
        # the direct vs128 launcher keeps the 256-row kernel its grid names (the single-stream order), correct here too
        import ctypes, math, torch
        q, k, v, qs, ks, vs = gpu_util.upload(inp, gpu)
        o2 = torch.full((B, S, H, 128), float("nan"), dtype=torch.bfloat16, device=gpu)
        a = lib.fill_args(o2.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), qs.data_ptr(), ks.data_ptr(), vs.data_ptr(),
                          B, H, HK, S, SK)
        st = torch.cuda.current_stream(gpu).cuda_stream
        assert lib.raw.fmha_mxfp8_launch_vs128(ctypes.byref(a), math.ceil(S / 256), H, B, st) == 0
        torch.cuda.synchronize()
        direct = o2.view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)
        single = oracle.emulate(inp, rows=rows)
        dcmp = gpu_util.compare_to_emulation(direct, single, inp, rows)
        print(f"[case] vs128 direct launcher {name} vs-single-stream-emulation={dcmp}", flush=True)
        assert dcmp["mean_abs"] <= 0.6 * max(ref_stats["mean_err"], 1e-6), dcmp
        assert dcmp["max_abs"] <= 0.05, dcmp



# Extension: the causal q-tile pairing (FMHA_FLAG_CAUSAL_PAIR, the reference's causal_pair, grid.rs:94-111) on the
# 128-row grid: block x runs query tiles x and T - 1 - x. Each tile is computed exactly as unpaired, so the output must
# be bit-identical to the unpaired launch; and it meets the causal bar against the emulation on every checked row.
# (name, B, H, HK, S, SK, path); T odd leaves the middle tile alone; S > SK has rows that see no key; SK < 512 runs
# the 256-thread t128 kernel (the LUT recipe); B4H8S2048 has more 128-row blocks than CUs, so "auto" pairs it.
PAIR_CASES = [
    ("B1H4S1000_SK1337", 1, 4, 4, 1000, 1337, "auto"),
    ("B1H2S1408_T11", 1, 2, 2, 1408, 1408, "auto"),
    ("B2H4HK1_S700_gqa4", 2, 4, 1, 700, 700, "auto"),
    ("S_gt_SK_B1H2S900_SK600", 1, 2, 2, 900, 600, "auto"),
    ("t128_lut_B1H2S512_SK384", 1, 2, 2, 512, 384, "t128"),
    ("B4H8S2048_auto_pairs", 4, 8, 8, 2048, 2048, "auto"),
    # paired by the automatic rule with at most 8 key tiles: the 256-thread single-wave kernel, paired or not
    ("B16H8S512_auto_pairs_single_wave", 16, 8, 8, 512, 512, "auto"),
    ("B8H8S1024_vs128_auto_pairs_single_wave", 8, 8, 8, 1024, 1024, "vs128"),
]


@pytest.mark.parametrize("case", PAIR_CASES, ids=[c[0] for c in PAIR_CASES])
def test_causal_pairing(gpu, case):
    name, B, H, HK, S, SK, path = case
    print(f"[case] causal pairing {name}", flush=True)
    inp = oracle.Inputs(B, H, S, SK, HK=HK, causal=True)
    big = B * H * S * SK > (1 << 24)
    paired, used, _ = gpu_util.run(inp, gpu, path=path, causal_pair="auto" if big else True)
    plain, used2, _ = gpu_util.run(inp, gpu, path=path, causal_pair=False)
    assert used == used2 and (path == "auto" or used[0] == path)
    assert not np.isnan(oracle.bf16_to_f32(paired)).any()
    np.testing.assert_array_equal(paired, plain)
    rows = oracle.first_and_last(S, 128) if big else S
    emu, ref_stats = _emulated_bar(inp, 0, rows=rows, path=used[0])
    stats = oracle.check_fp64(inp, paired, rows=rows)
    cmp = gpu_util.compare_to_emulation(paired, emu, inp, rows)
    fig, viol = gpu_util.causal_bar(inp, paired, emu, rows)
    print(f"[case] causal pairing {name} path={used} ours={stats} emulated={ref_stats} vs-emulation={cmp} causal-bar={fig}",
          flush=True)
    # Bad elements: on the large causal grids the hardware kernels can leave a few more elements outside the harness
    # tolerance than the exact emulation (B16H8S512: 13 against 9): the first rows' outputs rest on a few keys, whose
    # P the MFMA's inexact sums can carry across an e4m3 rounding step. causal_bar admits such an element only where
    # one step of one key's P explains its distance from the emulation, in at most 2 % of the rows.
    assert stats["bad"] <= ref_stats["bad"] + fig["extra"]
    assert stats["mean_err"] <= 1.10 * ref_stats["mean_err"] + 1e-7
    assert cmp["mean_abs"] <= 0.6 * max(ref_stats["mean_err"], 1e-6), cmp
    assert not viol, (viol, fig)


# Extension: KV-split workspace slots. A workspace of k times the reference's size is used as min(k, 4) slots taken in
# turn by consecutive calls; each slot holds a whole call's partials, so every call must give the bits of the
# one-slot call. The workspace is filled with NaN bytes first: a call reading another slot's (or no) partials would
# show as NaN or as a difference.
def test_workspace_slots(gpu):
    import torch
    inp = oracle.Inputs(1, 8, 512, 4096, seed_mix=11)
    print("[case] workspace slots B1H8S512_SK4096", flush=True)
    q, k, v, qs, ks, vs = gpu_util.upload(inp, gpu)
    B, H, S, SK = inp.B, inp.H, inp.S, inp.SK
    used = lib.select_path(B, H, S, SK)
    assert used[0] == "kvsplit"
    # (sized for the partials the entry writes with the fill, so that every workspace below runs the same partials)
    parts = lib.kv_partials(B, H, S, SK, used[1])
    need = lib.workspace_bytes(B, H, S, parts)
    turn = ctypes.c_uint32(0)
    st = torch.cuda.current_stream(gpu).cuda_stream

    def call(ws, nbytes):
        out = torch.full((B, S, H, 128), float("nan"), dtype=torch.bfloat16, device=gpu)
        p = lib.Params()
        p.o, p.q, p.k, p.v = out.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr()
        p.q_descale, p.k_descale, p.v_descale, p.lse = qs.data_ptr(), ks.data_ptr(), vs.data_ptr(), None
        p.bytes_q, p.bytes_k, p.bytes_v, p.bytes_o = ops._cap(q), ops._cap(k), ops._cap(v), ops._cap(out)
        p.bytes_q_descale, p.bytes_k_descale, p.bytes_v_descale = ops._cap(qs), ops._cap(ks), ops._cap(vs)
        p.B, p.H, p.HK, p.S, p.SK = B, H, inp.HK, S, SK
        p.path, p.splits = -1, 0
        p.ws_turn = ctypes.pointer(turn)
        ran = lib.run_auto(p, ws.data_ptr(), nbytes, st)
        assert ran == used and ran.partials == parts
        torch.cuda.synchronize()
        return out.view(torch.int16).cpu().numpy()

    one = torch.full((need,), 0xFF, dtype=torch.uint8, device=gpu)
    want = call(one, need)
    assert not np.isnan(oracle.bf16_to_f32(want.view(np.uint16))).any()
    stride = (need + 255) // 256 * 256
    four = torch.full((lib.WORKSPACE_SLOTS * stride,), 0xFF, dtype=torch.uint8, device=gpu)
    for i in range(2 * lib.WORKSPACE_SLOTS + 1):
        np.testing.assert_array_equal(call(four, four.numel()), want, err_msg=f"call {i}")


# Extension: the KV-split fill. With few blocks per chunk the one-call entry spreads each of the reference's chunks
# over up to 8 blocks (lib.kv_partials) and merges every block's partial (the combine with the splits spread over a
# block's 4 waves above 8 partials per row). Bar: the reference's statistics on its own chunks, and element-wise
# closeness to the emulation of the partials that ran; kv_fill=False runs the reference's chunks only.
FILL_CASES = [
    ("cfg5_B1H8S128_SK16384_split8", 1, 8, 8, 128, 16384, "kvsplit", 8),
    ("cfg5_tail_B1H8S128_SK16000_split8", 1, 8, 8, 128, 16000, "kvsplit", 8),
    ("auto_B1H8S512_SK32768", 1, 8, 8, 512, 32768, "auto", None),
    ("auto_gqa4_B1H8HK2_S256_SK8192", 1, 8, 2, 256, 8192, "auto", None),
]


@pytest.mark.parametrize("case", FILL_CASES, ids=[c[0] for c in FILL_CASES])
def test_parity_kv_fill(gpu, case):
    name, B, H, HK, S, SK, path, splits = case
    print(f"[case] kv fill {name}", flush=True)
    inp = oracle.Inputs(B, H, S, SK, HK=HK)
    chunks = gpu_util.chunks(inp, path, splits)
    out, used, _ = gpu_util.run(inp, gpu, path=path, splits=splits)
    ref_out, ref_used, _ = gpu_util.run(inp, gpu, path=path, splits=splits, kv_fill=False)
    assert used == ("kvsplit", chunks) and used.partials == lib.kv_partials(B, H, S, SK, chunks) and used.partials > chunks
    assert ref_used == ("kvsplit", chunks) and ref_used.partials == chunks
    rows = oracle.first_and_last(S, ROWS)
    emu, ref_stats = _emulated_bar(inp, used.partials, rows=rows, ref_splits=chunks)
    stats = oracle.check_fp64(inp, out, rows=rows)
    stats_chunks = oracle.check_fp64(inp, ref_out, rows=rows)
    cmp = gpu_util.compare_to_emulation(out, emu, inp, rows)
    print(f"[case] kv fill {name} ran={used} ours={stats} chunks-only={stats_chunks} emulated-reference={ref_stats} "
          f"vs-emulation={cmp}", flush=True)
    assert not np.isnan(oracle.bf16_to_f32(out)).any()
    for st in (stats, stats_chunks):
        assert st["bad"] <= ref_stats["bad"]
        assert st["mean_err"] <= 1.10 * ref_stats["mean_err"]
    assert cmp["mean_abs"] <= 0.6 * ref_stats["mean_err"], cmp
    assert cmp["max_abs"] <= 0.05, cmp


# The 128-row grids below the split-tile threshold (4 to 6 key tiles, no causal mask): the one-call entry runs them on
# the 256-thread t128 kernel, the reference's order. t128's shapes must give the direct t128 launcher's bits, and
# vs128's half-chip shapes the direct vs128 launcher's (the 256-row kernel takes every tile whole too); both meet the
# bar against the emulation of the reference's order.
SINGLE_WAVE_CASES = [
    ("t128_B1H8S512", 1, 8, 8, 512, 512, "t128"),
    ("t128_B2H8HK2_S700_SK700", 2, 8, 2, 700, 700, "t128"),
    ("t128_B1H4S300_SK600", 1, 4, 4, 300, 600, "t128"),
    ("vs128_B8H8S512", 8, 8, 8, 512, 512, "vs128"),
    ("vs128_B2H8S2048_SK768", 2, 8, 8, 2048, 768, "vs128"),
]


@pytest.mark.parametrize("case", SINGLE_WAVE_CASES, ids=[c[0] for c in SINGLE_WAVE_CASES])
def test_parity_128row_single_wave(gpu, case):
    name, B, H, HK, S, SK, path = case
    print(f"[case] single wave {name}", flush=True)
    assert not lib.uses_split_tiles(path, B, H, S, SK)
    inp = oracle.Inputs(B, H, S, SK, HK=HK)
    out, used, _ = gpu_util.run(inp, gpu, path=path)
    assert used == (path, 0)
    rows = S if B * H * S * SK <= 10_000_000 else oracle.first_and_last(S, 128)
    emu, ref_stats = _emulated_bar(inp, 0, rows=rows, path=path)
    stats = oracle.check_fp64(inp, out, rows=rows)
    cmp = gpu_util.compare_to_emulation(out, emu, inp, rows)
    print(f"[case] single wave {name} ours={stats} emulated-reference={ref_stats} vs-emulation={cmp}", flush=True)
    assert not np.isnan(oracle.bf16_to_f32(out)).any()
    assert stats["bad"] <= ref_stats["bad"]
    assert stats["mean_err"] <= 1.10 * ref_stats["mean_err"] + 1e-7
    assert cmp["mean_abs"] <= 0.6 * max(ref_stats["mean_err"], 1e-6), cmp
    assert cmp["max_abs"] <= 0.05, cmp
    np.testing.assert_array_equal(gpu_util.run_direct(inp, gpu, path), out)


def _random_cases(n=16, seed=20261202):
    """Seeded random shapes for the one-call entry's dispatch (every path it can pick, ragged S and SK, GQA, causal):
    sizes at which the oracle checks them in seconds."""
    rs = np.random.RandomState(seed)
    cases = []
    for i in range(n):
        H = int(rs.choice([1, 2, 4, 8]))
        HK = int(rs.choice([d for d in (1, 2, 4, 8) if d <= H and H % d == 0]))
        B = int(rs.randint(1, 4)) if H <= 4 else int(rs.randint(1, 3))
        S = int(rs.randint(1, 200)) if rs.rand() < 0.4 else int(rs.randint(200, 1300))
        SK = int(rs.randint(1, 300)) if rs.rand() < 0.3 else int(rs.randint(300, 2600))
        causal = bool(rs.rand() < 0.3)
        cases.append((f"rand{i}_B{B}H{H}HK{HK}_S{S}_SK{SK}" + ("_causal" if causal else ""), B, H, HK, S, SK, causal))
    # grids of more than 128 256-row blocks, where the dispatch picks the 256-row vs128 kernel
    for i in range(4):
        B = int(rs.randint(4, 9))
        HK = int(rs.choice([2, 4, 8]))
        S = int(rs.randint(1100, 2100))
        SK = int(rs.randint(200, 1300))
        causal = i % 2 == 1
        cases.append((f"randL{i}_B{B}H8HK{HK}_S{S}_SK{SK}" + ("_causal" if causal else ""), B, 8, HK, S, SK, causal))
    return cases


RANDOM_CASES = _random_cases()


@pytest.mark.parametrize("case", RANDOM_CASES, ids=[c[0] for c in RANDOM_CASES])
def test_parity_random_shapes(gpu, case):
    """The fixed cases' bars (test_parity, test_parity_causal) on seeded random shapes through the automatic
    dispatch."""
    name, B, H, HK, S, SK, causal = case
    print(f"[case] {name}", flush=True)
    inp = oracle.Inputs(B, H, S, SK, HK=HK, causal=causal)
    out, used, _ = gpu_util.run(inp, gpu)
    rows = S if S <= 128 else oracle.first_and_last(S, ROWS)
    used_splits = used.partials if used[0] == "kvsplit" else 0
    emu, ref_stats = _emulated_bar(inp, used_splits, rows=rows, path=used[0], ref_splits=gpu_util.chunks(inp))
    stats = oracle.check_fp64(inp, out, rows=rows)
    cmp = gpu_util.compare_to_emulation(out, emu, inp, rows)
    print(f"[case] {name} path={used} partials={used.partials} ours={stats} emulated-reference={ref_stats} "
          f"vs-emulation={cmp}", flush=True)
    assert not np.isnan(oracle.bf16_to_f32(out)).any(), "unwritten / NaN outputs"
    assert stats["bad"] <= ref_stats["bad"]
    assert stats["mean_err"] <= 1.10 * ref_stats["mean_err"] + 1e-7
    assert cmp["mean_abs"] <= 0.6 * max(ref_stats["mean_err"], 1e-6), cmp
    if causal:
        fig, viol = gpu_util.causal_bar(inp, out, emu, rows)
        assert not viol, (viol, fig)
        if S > SK:
            o = oracle.bf16_to_f32(out).reshape(B, S, H, 128)
            assert (o[:, : S - SK] == 0).all()
    else:
        assert cmp["max_abs"] <= 0.05, cmp


def _random_ext_cases(n=16, seed=77):
    """Seeded random combinations of the extensions (per-32-key V scales, the in-kernel softmax scale, f32 partials,
    causal) with a forced path, on random shapes."""
    rs = np.random.RandomState(seed)
    cases = []
    for i in range(n):
        H = int(rs.choice([1, 2, 4, 8]))
        HK = int(rs.choice([d for d in (1, 2, 4, 8) if d <= H and H % d == 0]))
        B = int(rs.randint(1, 3))
        S = int(rs.randint(1, 150)) if rs.rand() < 0.3 else int(rs.randint(150, 1100))
        SK = int(rs.randint(1, 400)) if rs.rand() < 0.3 else int(rs.randint(400, 2500))
        path = str(rs.choice(["vs128", "t128", "kvsplit"]))
        causal = path != "kvsplit" and rs.rand() < 0.4
        splits = int(rs.choice([2, 4, 8])) if path == "kvsplit" else None
        if splits:
            # validate (the reference's rule) refuses a split left without a key tile: the largest count that fits
            nt = (SK + 127) // 128
            while splits > 2 and (splits - 1) * -(-nt // splits) >= nt:
                splits //= 2
            if (splits - 1) * -(-nt // splits) >= nt:
                SK = max(SK, 257)
        opt = {"v_seq32": bool(rs.rand() < 0.5),
               "qk_scale": float(rs.choice([0.0, 0.3, 0.7, 1.3])),
               "partials": "fp32" if path == "kvsplit" and rs.rand() < 0.5 else "fp16"}
        tag = "".join(["_causal" if causal else "", "_vs32" if opt["v_seq32"] else "",
                       f"_c{opt['qk_scale']}" if opt["qk_scale"] else "", "_f32" if opt["partials"] == "fp32" else ""])
        cases.append((f"ext{i}_{path}{splits or ''}_B{B}H{H}HK{HK}_S{S}_SK{SK}{tag}", B, H, HK, S, SK, causal, path,
                      splits, opt))
    return cases


RANDOM_EXT_CASES = _random_ext_cases()


@pytest.mark.parametrize("case", RANDOM_EXT_CASES, ids=[c[0] for c in RANDOM_EXT_CASES])
def test_parity_random_extensions(gpu, case):
    """The extensions' bars (test_parity_v_seq32, test_parity_qk_scale, test_parity_f32_partials, the causal bar) on
    seeded random combinations."""
    name, B, H, HK, S, SK, causal, path, splits, opt = case
    print(f"[case] {name}", flush=True)
    inp = oracle.Inputs(B, H, S, SK, HK=HK, causal=causal, v_seq32=opt["v_seq32"], qk_scale=opt["qk_scale"])
    out, used, _ = gpu_util.run(inp, gpu, path=path, splits=splits, partials=opt["partials"])
    assert used[0] == path
    rows = S if S <= 128 else oracle.first_and_last(S, ROWS)
    used_splits = used.partials if used[0] == "kvsplit" else 0
    emu, ref_stats = _emulated_bar(inp, used_splits, rows=rows, path=used[0], ref_splits=gpu_util.chunks(inp, path, splits),
                                   f32_partials=opt["partials"] == "fp32")
    stats = oracle.check_fp64(inp, out, rows=rows)
    cmp = gpu_util.compare_to_emulation(out, emu, inp, rows)
    print(f"[case] {name} path={used} partials={used.partials} ours={stats} emulated-reference={ref_stats} "
          f"vs-emulation={cmp}", flush=True)
    assert not np.isnan(oracle.bf16_to_f32(out)).any(), "unwritten / NaN outputs"
    assert stats["bad"] <= ref_stats["bad"]
    assert stats["mean_err"] <= 1.10 * ref_stats["mean_err"] + 1e-7
    assert cmp["mean_abs"] <= 0.6 * max(ref_stats["mean_err"], 1e-6), cmp
    if causal:
        fig, viol = gpu_util.causal_bar(inp, out, emu, rows)
        assert not viol, (viol, fig)
        if S > SK:
            o = oracle.bf16_to_f32(out).reshape(B, S, H, 128)
            assert (o[:, : S - SK] == 0).all()
    else:
        assert cmp["max_abs"] <= 0.05, cmp
