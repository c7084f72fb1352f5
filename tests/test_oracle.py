"""CPU tests that pin the oracle (oracle/mxfp8_oracle.c) before it is trusted as the checker.

Each oracle function is checked against something it does not itself compute:
  * the reference's published per-shape accuracy and path choice (docs/perf-matrix.md:29-53; REF_DATA=normal,
    64 rows): generator + recipe emulation + fp64 check + dispatch together reproduce every published figure;
  * what gfx950 returned for the conversion instructions and the scaled MFMA (tests/golden/hw_probe.npz, written
    by tests/golden/make_hw_fixture.py on an MI355X);
  * independent implementations of the mathematics (torch's e4m3 codec, numpy float64 attention, the closed-form
    LSE-weighted average of the combine);
  * invariants (E8M0 block rule, split-vs-full ULP gate of tests/gpu/ref_host.cpp:616-636, determinism).
"""
import os

import numpy as np
import pytest
import torch

import oracle

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden", "hw_probe.npz")
D = 128

# docs/perf-matrix.md:31-55: (B, H, S, SK, gqa, path, published bad, published mean_err) of the reference kernels
PUBLISHED = [
    (1, 8, 512, 512, 1, "t128", 0, 1.74e-03), (1, 8, 1024, 1024, 1, "t128", 0, 1.25e-03),
    (1, 8, 2048, 2048, 1, "kvsplit", 0, 8.86e-04), (1, 8, 4096, 4096, 1, "kvsplit", 0, 6.41e-04),
    (1, 8, 8192, 8192, 1, "vs128", 0, 4.58e-04), (2, 8, 512, 512, 1, "t128", 0, 1.74e-03),
    (2, 8, 1024, 1024, 1, "t128", 0, 1.26e-03), (2, 8, 2048, 2048, 1, "vs128", 0, 9.07e-04),
    (2, 8, 4096, 4096, 1, "vs128", 0, 6.43e-04), (2, 8, 8192, 8192, 1, "vs128", 0, 4.57e-04),
    (4, 8, 512, 512, 1, "t128", 0, 1.73e-03), (4, 8, 1024, 1024, 1, "vs128", 0, 1.26e-03),
    (4, 8, 2048, 2048, 1, "vs128", 0, 9.06e-04), (4, 8, 4096, 4096, 1, "vs128", 0, 6.43e-04),
    (4, 8, 8192, 8192, 1, "vs128", 0, 4.59e-04), (8, 8, 512, 512, 1, "vs128", 0, 1.74e-03),
    (8, 8, 1024, 1024, 1, "vs128", 0, 1.26e-03), (8, 8, 2048, 2048, 1, "vs128", 0, 9.02e-04),
    (8, 8, 4096, 4096, 1, "vs128", 0, 6.46e-04), (8, 8, 8192, 8192, 1, "vs128", 0, 4.59e-04),
    (1, 8, 2048, 2048, 2, "kvsplit", 0, 8.92e-04), (1, 8, 2048, 2048, 4, "kvsplit", 0, 8.85e-04),
    (1, 8, 1000, 1000, 1, "t128", 0, 1.28e-03), (1, 8, 2048, 1337, 1, "t128", 0, 1.10e-03),
    (1, 8, 1000, 1337, 1, "t128", 0, 1.10e-03),
]
# the emulation cost grows with B * SK; the larger shapes run with FMHA_ORACLE_FULL=1 (about 2 minutes more)
_FULL = os.environ.get("FMHA_ORACLE_FULL") == "1"
_PUB_CASES = [c for c in PUBLISHED if _FULL or c[0] * c[3] <= 8192]


@pytest.fixture(scope="module")
def hw():
    return np.load(GOLDEN)


# ------------------------------------------------------------------ conversions


def test_e4m3_decode_matches_torch():
    """ref_host.cpp:26-33 decode of all 256 bytes == torch's float8_e4m3fn, except the NaN bytes which decode to 0."""
    L = oracle.lib()
    b = np.arange(256, dtype=np.uint8)
    ours = np.array([L.mxo_e4m3_decode(int(x)) for x in b])
    ref = torch.from_numpy(b).view(torch.float8_e4m3fn).float().numpy().astype(np.float64)
    nan = np.isnan(ref)
    assert nan.sum() == 2 and set(b[nan]) == {0x7F, 0xFF}
    np.testing.assert_array_equal(ours[~nan], ref[~nan])
    assert (ours[nan] == 0).all()


def test_e4m3_encode_matches_torch():
    """RNE e4m3 encoder saturating at 448 (ref_host.cpp:216-228) == torch's RNE cast of the value clamped to +-448."""
    L = oracle.lib()
    rng = np.random.default_rng(3)
    grid = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    grid = grid[np.isfinite(grid)]
    mids = (np.sort(grid)[1:] + np.sort(grid)[:-1]) / 2
    x = np.concatenate([grid, mids, np.nextafter(mids, np.float32(1e9)), np.nextafter(mids, np.float32(-1e9)),
                        rng.standard_normal(4000) * 50, rng.uniform(-600, 600, 2000), [449.0, -1e6, 1e-9, -0.0]]).astype(np.float32)
    ours = np.array([L.mxo_e4m3_encode_sat(float(v)) for v in x], np.uint8)
    ref = torch.from_numpy(np.clip(x, -448, 448)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    # -0 and +0 both decode to 0: compare values, then the bytes of everything non-zero
    dv = lambda a: torch.from_numpy(a).view(torch.float8_e4m3fn).float().numpy()
    np.testing.assert_array_equal(dv(ours), dv(ref))


def test_cvt_bf16_fp8_matches_hardware(hw):
    """v_cvt_scalef32_pk_fp8_bf16 restatement == gfx950 on every bf16 pattern at the two P scales (1.0, 0.25)."""
    L = oracle.lib()
    for si, scale in enumerate((1.0, 0.25)):
        ours = np.array([L.mxo_cvt_bf16_fp8(u, scale) for u in range(65536)], np.uint8)
        got = hw["cvt"][si]
        bad = np.nonzero(ours != got)[0]
        assert bad.size == 0, f"scale {scale}: {bad.size} mismatches, first bf16 0x{bad[0]:04x}: ours 0x{ours[bad[0]]:02x} hw 0x{got[bad[0]]:02x}"


def test_pknorm_matches_hardware(hw):
    """v_cvt_pknorm_u16_f32 restatement (RNE of 65535 clamp(x, 0, 1)) == gfx950 on the probe inputs."""
    L = oracle.lib()
    x, got = hw["pk_in"], hw["pk_out"]
    ours = np.array([L.mxo_pknorm_u16(float(v)) for v in x], np.uint16)
    bad = np.nonzero(ours != got)[0]
    assert bad.size == 0, f"{bad.size} mismatches, first x={x[bad[0]]!r}: ours {ours[bad[0]]} hw {got[bad[0]]}"


def test_pknorm_closed_form_all_u16():
    """pknorm(k / 65535) == k for every u16 k (the round trip the exp2 trick relies on)."""
    L = oracle.lib()
    k = np.arange(65536)
    x = (k / 65535.0).astype(np.float32)
    ours = np.array([L.mxo_pknorm_u16(float(v)) for v in x], np.int64)
    np.testing.assert_array_equal(ours, k)


def test_f16_roundtrip_matches_numpy():
    L = oracle.lib()
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.standard_normal(3000) * 10, rng.uniform(-65000, 65000, 500), [0.0, -0.0, 65504.0, 1e-8]]).astype(np.float32)
    ours = np.array([L.mxo_f32_to_f16(float(v)) for v in x], np.uint16)
    np.testing.assert_array_equal(ours, x.astype(np.float16).view(np.uint16))
    back = np.array([L.mxo_f16_to_f32(int(h)) for h in ours], np.float32)
    np.testing.assert_array_equal(back, ours.view(np.float16).astype(np.float32))


def _mfma_reference(a, b, sa, sb, c):
    """fp64 model of v_mfma_scale_f32_32x32x64_f8f6f4 (e4m3 x e4m3, op_sel 0) in register layout: lane l holds row
    (A) / column (B) l % 32, bytes 0-15 = k 16 (l / 32) + j, bytes 16-31 = k 32 + 16 (l / 32) + j; the E8M0 scale of
    k-block kb of row r is byte 0 of lane r + 32 kb; D value r of lane l = row 8 (r / 4) + 4 (l / 32) + r % 4,
    column l % 32; D = sum_k 2^(sa - 127) A 2^(sb - 127) B + C."""
    dec = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy().astype(np.float64)
    A = np.zeros((32, 64)); Bm = np.zeros((64, 32)); SA = np.zeros((32, 2)); SB = np.zeros((32, 2))
    for l in range(64):
        r, h = l % 32, l // 32
        for j in range(16):
            A[r, 16 * h + j] = dec[a[l, j]]; A[r, 32 + 16 * h + j] = dec[a[l, 16 + j]]
            Bm[16 * h + j, r] = dec[b[l, j]]; Bm[32 + 16 * h + j, r] = dec[b[l, 16 + j]]
    for r in range(32):
        for kb in range(2):
            SA[r, kb] = 2.0 ** (int(sa[r + 32 * kb]) - 127); SB[r, kb] = 2.0 ** (int(sb[r + 32 * kb]) - 127)
    terms = np.zeros((32, 32, 64))
    for kb in range(2):
        ks = slice(32 * kb, 32 * kb + 32)
        terms[:, :, ks] = (A[:, None, ks] * SA[:, None, kb:kb + 1]) * (Bm.T[None, :, ks] * SB[None, :, kb:kb + 1])
    full = terms.sum(-1)
    mag = np.abs(terms).sum(-1)
    d = np.zeros((64, 16)); m = np.zeros((64, 16))
    for l in range(64):
        for r in range(16):
            i, j = 8 * (r // 4) + 4 * (l // 32) + r % 4, l % 32
            d[l, r] = full[i, j] + c[l, r]
            m[l, r] = mag[i, j] + abs(c[l, r])
    return d, m


def test_scaled_mfma_semantics_match_hardware(hw):
    """The MFMA operand / scale / result layout and the 2^(s - 127) E8M0 semantics the kernels and the oracle assume
    (a transposed operand or a mis-assigned scale lane gives errors of the order of the values themselves). The
    hardware sum is not exact: up to ~3e-4 of the summed magnitudes is allowed."""
    d, mag = _mfma_reference(hw["mfma_a"], hw["mfma_b"], hw["mfma_sa"], hw["mfma_sb"], hw["mfma_c"].astype(np.float64))
    got = hw["mfma_d"].astype(np.float64)
    err = np.abs(got - d)
    assert (err <= 1e-3 * mag + 1e-30).all(), f"max rel {np.max(err / (mag + 1e-30)):.3g}"
    assert np.median(err / (mag + 1e-30)) < 1e-4
    # negative control: the same model with the roles of the two operands exchanged (a transposed product) is far off
    d_t, mag_t = _mfma_reference(hw["mfma_b"], hw["mfma_a"], hw["mfma_sb"], hw["mfma_sa"], hw["mfma_c"].astype(np.float64))
    assert np.median(np.abs(got - d_t) / (mag_t + 1e-30)) > 1e-2


# ------------------------------------------------------------------ generator, dispatch, split ranges


def test_generator_e8m0_block_rule():
    """ref_host.cpp:239-251: E8M0 = floor(log2 amax) - 8 + 127, so every non-zero 32-element block's largest
    e4m3 magnitude lies in [256, 448] (448 = saturation of [448, 512))."""
    inp = oracle.Inputs(1, 2, 64, 96)
    dec = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    for x in (inp.q, inp.k):
        blk = np.abs(dec[x.reshape(-1, 32)])
        mx = blk.max(1)
        assert ((mx >= 256) & (mx <= 448)).all()


def test_generator_deterministic_and_seeded():
    a, b = oracle.Inputs(1, 2, 32, 48), oracle.Inputs(1, 2, 32, 48)
    c = oracle.Inputs(1, 2, 32, 48, seed_mix=99)
    assert (a.q == b.q).all() and (a.k == b.k).all() and (a.v == b.v).all() and a.vdescale == b.vdescale
    assert (a.q != c.q).any()


@pytest.mark.parametrize("case", PUBLISHED, ids=[f"B{c[0]}H{c[1]}S{c[2]}SK{c[3]}g{c[4]}" for c in PUBLISHED])
def test_dispatch_matches_published_paths(case):
    B, H, S, SK, g, path = case[:6]
    assert oracle.select_path(B, H, S, SK)[0] == path


def test_dispatch_closed_form():
    """dispatch.rs:494-511 on a grid: split 4 / split 2 / t128 / vs128 by blocks256 and ntiles."""
    for B in (1, 2, 4, 8):
        for H in (1, 8, 16, 32):
            for S in (1, 128, 256, 300, 1024, 2048, 8192):
                for SK in (1, 129, 2048, 4096, 16000, 16384):
                    b256 = -(-S // 256) * H * B
                    nt = -(-SK // 128)
                    path, sp = oracle.select_path(B, H, S, SK)
                    if nt >= 16 and b256 <= 64:
                        assert (path, sp) == ("kvsplit", 4)
                    elif nt >= 32 and b256 <= 128:
                        assert (path, sp) == ("kvsplit", 2)
                    else:
                        assert path == ("t128" if b256 <= 64 else "vs128")


def test_split_range_covers_keys_once():
    """components.rs:58-74: split s owns tiles [s tps, min(ntiles, (s + 1) tps)); together they cover [0, SK)."""
    for SK in (1, 100, 128, 129, 1337, 2048, 16000, 16384):
        for splits in (2, 4, 8):
            seen = np.zeros(SK, int)
            nt = -(-SK // 128)
            tps = -(-nt // splits)
            for s in range(splits):
                lo, n = oracle.split_range(SK, splits, s)
                assert lo == s * tps * 128
                if n > 0:   # a split past the last tile has no keys (kv_eff <= 0)
                    seen[lo:lo + n] += 1
            assert (seen == 1).all()


# ------------------------------------------------------------------ fp64 check / fp32 baseline vs numpy


def _numpy_attention(inp, rows):
    dec = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy().astype(np.float64)
    dec[[0x7F, 0xFF]] = 0.0
    B, H, HK, S, SK = inp.B, inp.H, inp.HK, inp.S, inp.SK
    q = dec[inp.q].reshape(B, S, H, 4, 32) * 2.0 ** (inp.qs[: B * S * H * 4].reshape(B, S, H, 4, 1).astype(np.float64) - 127)
    k = dec[inp.k].reshape(B, SK, HK, 4, 32) * 2.0 ** (inp.ks[: B * SK * HK * 4].reshape(B, SK, HK, 4, 1).astype(np.float64) - 127)
    if inp.vs32 is not None:   # extension: one E8M0 per 32 keys per column
        vsc = 2.0 ** (inp.vs32.reshape(B, -1, HK, D).astype(np.float64) - 127)
        v = dec[inp.v].reshape(B, SK, HK, D) * np.repeat(vsc, 32, axis=1)[:, :SK]
    else:
        v = dec[inp.v].reshape(B, SK, HK, D) * inp.vdescale
    q, k = q.reshape(B, S, H, D), k.reshape(B, SK, HK, D)
    g = H // HK
    # the in-kernel softmax scale (extension): base-2 scores times c = f32(scale) f32(log2 e), rounded to f32
    c = float(np.float32(inp.qk_scale) * np.float32(1.4426950408889634)) if inp.qk_scale > 0 else 1.0
    out = np.zeros((B, rows, H, D))
    for b in range(B):
        for h in range(H):
            s = q[b, :rows, h] @ k[b, :, h // g].T * np.log(2.0) * c
            if inp.causal:
                i = np.arange(rows)[:, None]; t = np.arange(SK)[None, :]
                s = np.where(t <= i + SK - S, s, -np.inf)
            s = s - s.max(1, keepdims=True)
            p = np.exp(s)
            out[b, :, h] = (p / p.sum(1, keepdims=True)) @ v[b, :, h // g]
    return out


@pytest.mark.parametrize("causal,v_seq32,scale", [(False, False, 0.0), (True, False, 0.0), (False, True, 0.0),
                                                 (True, True, 0.7), (False, False, 1.3)])
def test_check_fp64_matches_numpy(causal, v_seq32, scale):
    """ref_host.cpp:436-471 statistics (bad = |err| > 0.05 + 0.05 |ref|, mean |err|) of a given output == the same
    statistics computed from numpy float64 attention (also with the per-32-key V scales and the in-kernel softmax
    scale of the extensions)."""
    inp = oracle.Inputs(2, 4, 40, 70, HK=2, causal=causal, v_seq32=v_seq32, qk_scale=scale)
    rows = 24
    ref = _numpy_attention(inp, rows)
    rng = np.random.default_rng(1)
    outf = np.zeros((inp.B, inp.S, inp.H, D), np.float32)
    outf[:, :rows] = ref + rng.standard_normal(ref.shape) * 0.03
    out = (outf.view(np.uint32) >> 16).astype(np.uint16)   # truncation to bf16 is fine: the statistic sees these bits
    got = oracle.check_fp64(inp, out, rows=rows)
    o = oracle.bf16_to_f32(out).reshape(outf.shape)[:, :rows].astype(np.float64)
    err = np.abs(o - ref)
    assert got["checked"] == err.size
    assert got["bad"] == int((err > 0.05 + 0.05 * np.abs(ref)).sum())
    assert abs(got["mean_err"] - err.mean()) <= 1e-9 * max(1.0, err.mean())


@pytest.mark.parametrize("causal,v_seq32,scale", [(True, True, 0.7), (False, False, 1.3), (True, False, 0.0)])
def test_gpu_util_float64_matches_numpy(causal, v_seq32, scale):
    """The GPU tests' float64 attention (tests/gpu_util.py: causal_rows under the causal bar, fp64_rows under the
    gate bar) == numpy float64 attention, with the extensions' per-32-key V scales and in-kernel softmax scale."""
    from tests import gpu_util
    inp = oracle.Inputs(2, 4, 40, 70, HK=2, causal=causal, v_seq32=v_seq32, qk_scale=scale)
    ref = _numpy_attention(inp, inp.S)
    if causal:
        got, vis, _ = gpu_util.causal_rows(inp, inp.S)
        assert (vis == np.clip(np.arange(inp.S) + inp.SK - inp.S + 1, 0, inp.SK)).all()
    else:
        got, _, _ = gpu_util.fp64_rows(inp, inp.S)
    np.testing.assert_allclose(got, ref, rtol=1e-9, atol=1e-12)


@pytest.mark.parametrize("causal,v_seq32", [(False, False), (True, False), (False, True)])
def test_attention_fp32_matches_numpy(causal, v_seq32):
    inp = oracle.Inputs(1, 4, 50, 90, HK=4, causal=causal, v_seq32=v_seq32)
    _, out = oracle.attention_fp32(inp, rows=0)
    ref = _numpy_attention(inp, inp.S)
    np.testing.assert_allclose(out.reshape(ref.shape), ref, atol=2e-5, rtol=1e-4)


# ------------------------------------------------------------------ the recipe emulation


@pytest.mark.parametrize("case", _PUB_CASES, ids=[f"B{c[0]}H{c[1]}S{c[2]}SK{c[3]}g{c[4]}" for c in _PUB_CASES])
def test_emulation_reproduces_published_accuracy(case):
    """Generator + recipe emulation + fp64 check reproduce the reference kernel's published bad / mean_err on the same
    shape and data (published to 3 significant figures; the reference's own MFMA summation adds a little spread)."""
    B, H, S, SK, g, path, bad, mean = case
    inp = oracle.Inputs(B, H, S, SK, HK=H // g)
    p, sp = oracle.select_path(B, H, S, SK)
    out = oracle.emulate(inp, splits=sp if p == "kvsplit" else 0, rows=64)
    st = oracle.check_fp64(inp, out, rows=64)
    assert st["bad"] == bad
    assert abs(st["mean_err"] / mean - 1.0) <= 0.012, st


def test_emulation_recipe_matters():
    """The published mean_err separates the recipes: the short-sequence (LUT) figure at S=SK=512 is not reproduced by
    the lazy recipe's statistics of a long sequence, and vice versa (guards against a test that passes for any
    output): the emulated error of B1H8S512 is 1.74e-3, of B1H8S8192 4.58e-4."""
    a = oracle.check_fp64(oracle.Inputs(1, 8, 512, 512), oracle.emulate(oracle.Inputs(1, 8, 512, 512), rows=64), rows=64)
    assert abs(a["mean_err"] / 1.74e-3 - 1) < 0.012
    # a zero output must fail the bar by far
    inp = oracle.Inputs(1, 8, 512, 512)
    z = oracle.check_fp64(inp, np.zeros(inp.out_elems, np.uint16), rows=64)
    assert z["mean_err"] > 5 * a["mean_err"]


def test_emulation_deterministic():
    inp = oracle.Inputs(1, 2, 256, 640)
    a = oracle.emulate(inp, rows=32, threads=1)
    b = oracle.emulate(inp, rows=32, threads=4)
    np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("splits", [2, 4, 8, 16, 32])
def test_split_matches_full_statistically(splits):
    """Each KV split starts its own softmax reference (b = 64), so its fp8 P rounding differs from the full-sequence
    kernel's and the outputs differ at the quantisation-noise level, not bit for bit: the split output must be at
    least as accurate as the full one (fp64 check) and differ from it by less than that error."""
    inp = oracle.Inputs(1, 2, 64, 4096 - 50)
    full_o = oracle.emulate(inp, splits=0, rows=64)
    sp_o = oracle.emulate(inp, splits=splits, rows=64)
    st_full, st_sp = oracle.check_fp64(inp, full_o, rows=64), oracle.check_fp64(inp, sp_o, rows=64)
    # (no less accurate; splits of fewer than 4 key tiles take the exact-rebasing recipe and come out more accurate)
    assert st_sp["bad"] == 0 and st_sp["mean_err"] / st_full["mean_err"] < 1.1
    diff = np.abs(oracle.bf16_to_f32(full_o).astype(np.float64) - oracle.bf16_to_f32(sp_o))
    assert diff.mean() < 1.5 * st_full["mean_err"] * (inp.S / 64)


@pytest.mark.parametrize("splits", [4, 32])
def test_combine_closed_form(splits):
    """epilogue.rs:89-167 streaming merge == the closed form sum_s 2^lse_s O_s / sum_s 2^lse_s (to bf16 rounding);
    a split with lse = -1e30 (no keys) has weight 0."""
    rng = np.random.default_rng(11)
    rows = 37
    ohat = rng.standard_normal((splits, rows, D)).astype(np.float16)
    lse = (rng.standard_normal((splits, rows)) * 6 - 3).astype(np.float32)
    lse[2, 5] = -1e30
    out = oracle.bf16_to_f32(oracle.combine(ohat.view(np.uint16), lse, rows, splits)).reshape(rows, D).astype(np.float64)
    w = np.exp2(lse.astype(np.float64) - lse.max(0))
    w[lse < -1e29] = 0.0
    ref = (w[:, :, None] * ohat.astype(np.float64)).sum(0) / w.sum(0)[:, None]
    assert (np.abs(out - ref) <= np.abs(ref) * 2.0 ** -8 + 1e-6).all()


def test_emulated_partials_combine_to_emulated_output():
    """The emulated split partials merged by the combine give the emulated split output, bit for bit."""
    inp = oracle.Inputs(1, 2, 40, 1000)
    splits = 4
    out, ohat, lse = oracle.emulate(inp, splits=splits, rows=0, partials=True)
    merged = oracle.combine(ohat, lse, inp.B * inp.S * inp.H, splits)
    np.testing.assert_array_equal(merged, out)


def test_combine_f32_closed_form():
    """The combine on f32 partial rows (extension) is the same streaming merge: the closed form to bf16 rounding, and
    on fp16-representable rows it equals the fp16 combine bit for bit."""
    rng = np.random.default_rng(12)
    rows, splits = 29, 8
    ohat = rng.standard_normal((splits, rows, D)).astype(np.float32)
    lse = (rng.standard_normal((splits, rows)) * 6 - 3).astype(np.float32)
    lse[3, 7] = -1e30
    out = oracle.bf16_to_f32(oracle.combine(ohat, lse, rows, splits)).reshape(rows, D).astype(np.float64)
    w = np.exp2(lse.astype(np.float64) - lse.max(0))
    w[lse < -1e29] = 0.0
    ref = (w[:, :, None] * ohat.astype(np.float64)).sum(0) / w.sum(0)[:, None]
    assert (np.abs(out - ref) <= np.abs(ref) * 2.0 ** -8 + 1e-6).all()
    h = ohat.astype(np.float16)
    np.testing.assert_array_equal(oracle.combine(h.astype(np.float32), lse, rows, splits),
                                  oracle.combine(h.view(np.uint16), lse, rows, splits))


def test_emulated_f32_partials():
    """Emulated KV split with f32 partial rows (extension): the rows are the fp16 rows before their rounding (within
    one fp16 rounding step), they combine to the emulated output bit for bit, and the result is at least as close to
    fp64 attention as the fp16 path."""
    inp = oracle.Inputs(1, 2, 40, 1000)
    splits = 4
    out16, oh16, lse16 = oracle.emulate(inp, splits=splits, rows=0, partials=True)
    out32, oh32, lse32 = oracle.emulate(inp, splits=splits, rows=0, partials=True, f32_partials=True)
    np.testing.assert_array_equal(lse16, lse32)
    assert oh32.dtype == np.float32
    np.testing.assert_array_equal(oh32.astype(np.float16).view(np.uint16), oh16)
    np.testing.assert_array_equal(oracle.combine(oh32, lse32, inp.B * inp.S * inp.H, splits), out32)
    e16 = oracle.check_fp64(inp, out16, rows=inp.S)
    e32 = oracle.check_fp64(inp, out32, rows=inp.S)
    assert e32["bad"] <= e16["bad"] and e32["mean_err"] <= e16["mean_err"] * 1.01


def test_emulation_v_seq32_scales():
    """Per-32-key V scales (extension) in the recipe emulation: raising every scale by one binade doubles the output
    exactly; raising only block 1 of column 5 changes only column 5; the statistics stay those of the per-tensor V (same
    data, re-quantised)."""
    inp = oracle.Inputs(1, 2, 48, 100, v_seq32=True)
    base = oracle.bf16_to_f32(oracle.emulate(inp, rows=0)).reshape(1, 48, 2, D)
    keep = inp.vs32.copy()
    inp.vs32 = keep + 1
    np.testing.assert_array_equal(oracle.bf16_to_f32(oracle.emulate(inp, rows=0)).reshape(base.shape), 2 * base)
    sc = keep.copy().reshape(1, -1, 2, D)
    sc[:, 1, :, 5] += 1
    inp.vs32 = sc.reshape(-1)
    got = oracle.bf16_to_f32(oracle.emulate(inp, rows=0)).reshape(base.shape)
    changed = got != base
    assert changed[..., 5].any() and not np.delete(changed, 5, axis=-1).any()
    inp.vs32 = keep
    ref = oracle.Inputs(1, 2, 48, 100)
    e32 = oracle.check_fp64(inp, oracle.emulate(inp, rows=0), rows=48)
    et = oracle.check_fp64(ref, oracle.emulate(ref, rows=0), rows=48)
    assert e32["bad"] == et["bad"] == 0 and 0.7 * et["mean_err"] < e32["mean_err"] < 1.4 * et["mean_err"]


# ------------------------------------------------------------------ quantisers of bf16 inputs

_E4M3 = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()


def _f32_to_bf16_bits(a):
    return (np.asarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def test_quant_rows_reproduces_the_generator():
    """The generator's own output (q, E8M0) dequantised to bf16 (exact: 4 significant bits) and quantised again by
    the restated rule gives back the generator's bytes. Its blocks' largest element lies in [256, 448], so the
    rule must return the same exponent; the only change allowed is -0 (0x80, a negative value that rounded to
    zero) coming back as +0, since the generator's sign byte is `x < 0` (ref_host.cpp:219)."""
    inp = oracle.Inputs(2, 4, 96, 80, HK=2)
    for x, s in ((inp.q, inp.qs), (inp.k, inp.ks)):
        rows = x.size // D
        sc = s[: rows * 4].reshape(rows, 4)
        val = _E4M3[x.reshape(rows, 4, 32)] * np.exp2(sc.astype(np.float64) - 127)[:, :, None]
        bits = _f32_to_bf16_bits(val.astype(np.float32))
        assert np.array_equal(oracle.bf16_to_f32(bits).reshape(val.shape), val.astype(np.float32))
        q2, s2 = oracle.quant_rows_bf16(bits)
        assert np.array_equal(s2, sc.reshape(-1))
        want = np.where(x == 0x80, 0, x)
        assert np.array_equal(q2, want)


def test_quant_rows_known_answers():
    """Hand-evaluated ref_host.cpp:243-247 on single blocks. amax 500 = 1.95 2^8: E8M0 = 8 - 8 + 127 = 127 and 500
    saturates to 448 (0x7E); the GEMM family's ceil(log2(amax / 448)) rule would give 128 and 250 -> 0x77 instead.
    amax 256: 127, 256 -> 0x78. amax 2^-130 (a bf16 subnormal): clamps to E8M0 0, element 2^-130 2^127 = 2^-3 ->
    0x20. An all-zero block: E8M0 0, bytes 0."""
    x = np.zeros((1, D), np.float32)
    x[0, 0], x[0, 1] = 500.0, -1.0
    x[0, 32] = 256.0
    x[0, 64] = 2.0 ** -130
    q, s = oracle.quant_rows_bf16(_f32_to_bf16_bits(x))
    assert list(s) == [127, 127, 0, 0]
    assert q[0] == 0x7E and q[1] == 0xB8 and q[32] == 0x78 and q[64] == 0x20
    assert (q[96:] == 0).all()
    # the multiplier applies before the block maximum: 2 x 250 = 500 again
    x2 = x.copy()
    x2[0, 0] = 250.0
    q2, s2 = oracle.quant_rows_bf16(_f32_to_bf16_bits(x2), 2.0)
    assert s2[0] == 127 and q2[0] == 0x7E


def test_quant_tensor_closed_form():
    """ref_host.cpp:248-251 with amax 448 (descale exactly 1) and 896 (descale 2): e4m3 grid values come back as
    their own bytes, midpoints between neighbours go to the even byte, magnitudes past 448 saturate."""
    pos = _E4M3[:127].astype(np.float32)
    mids = ((pos[:-1] + pos[1:]) / 2).astype(np.float32)
    exact_mids = mids[_f32_to_bf16_bits(mids).astype(np.uint32) << 16 == mids.view(np.uint32)]
    for scale in (1.0, 2.0):
        x = np.concatenate([pos, -pos, exact_mids, [448.0]]).astype(np.float32) * scale
        x = np.concatenate([x, np.zeros((-x.size) % 8, np.float32)])
        q, d = oracle.quant_tensor_bf16(_f32_to_bf16_bits(x))
        assert d == np.float32(scale)
        n = pos.size
        assert np.array_equal(q[:n], np.arange(127))
        assert np.array_equal(q[n:2 * n], np.where(np.arange(127) == 0, 0, np.arange(127) | 0x80))
        i = np.searchsorted(pos, exact_mids)
        assert np.array_equal(q[2 * n:2 * n + exact_mids.size], np.where(i % 2 == 0, i, i - 1))
    q, d = oracle.quant_tensor_bf16(_f32_to_bf16_bits(np.array([1000.0, -1.0, 0, 0, 0, 0, 0, 0], np.float32)))
    assert d == np.float32(1000.0 / 448.0) and q[0] == 0x7E


@pytest.mark.parametrize("B,SK,HK", [(1, 64, 1), (2, 45, 3)])
def test_quant_seq32_is_rows_rule_on_transposed_blocks(B, SK, HK):
    """Blocks along the sequence = the rows rule applied to the transposed [column, 32 keys] block (zero-padded
    keys past a ragged end change no maximum)."""
    rng = np.random.default_rng(SK)
    x = (rng.standard_normal((B, SK, HK, D)) * np.exp(rng.uniform(-8, 8, (B, SK, HK, D)))).astype(np.float32)
    bits = _f32_to_bf16_bits(x)
    q, s = oracle.quant_seq32_bf16(bits, B, SK, HK)
    nb = (SK + 31) // 32
    pad = np.zeros((B, nb * 32, HK, D), np.uint16)
    pad[:, :SK] = bits
    t = pad.reshape(B, nb, 32, HK, D).transpose(0, 1, 3, 4, 2)          # [B, nb, HK, D, 32 keys]
    qr, sr = oracle.quant_rows_bf16(t.reshape(-1, 128))                  # 4 columns of 32 keys per row of 128
    assert np.array_equal(s, sr)
    qt = qr.reshape(B, nb, HK, D, 32).transpose(0, 1, 4, 2, 3).reshape(B, nb * 32, HK, D)[:, :SK]
    assert np.array_equal(q.reshape(B, SK, HK, D), qt)


def test_split_tile_order_rule():
    """The split-tile order (extension: the library's KV split on blocks of at most 128 query rows) changes only the
    rows of such blocks: with S = 300 the rows of block 0 (300 valid rows) are bit-identical to the reference's order,
    rows 256..299 (44 valid rows) are not. Full-sequence emulation (the t128 path's split-tile kernel) takes every row
    in the split-tile order, except with the LUT recipe (fewer than 4 key tiles), which keeps the reference's."""
    inp = oracle.Inputs(1, 2, 300, 1000)
    ref = oracle.emulate(inp, splits=2, rows=0).reshape(1, 300, 2, D)
    st = oracle.emulate(inp, splits=2, rows=0, split_tiles=True).reshape(ref.shape)
    np.testing.assert_array_equal(st[:, :256], ref[:, :256])
    assert (st[:, 256:] != ref[:, 256:]).any()
    full = oracle.emulate(inp, rows=0).reshape(ref.shape)
    full_st = oracle.emulate(inp, rows=0, split_tiles=True).reshape(ref.shape)
    assert (full_st != full).mean() > 0.3
    lut = oracle.Inputs(1, 2, 300, 300)   # 3 key tiles: the LUT recipe
    np.testing.assert_array_equal(oracle.emulate(lut, rows=0, split_tiles=True), oracle.emulate(lut, rows=0))


@pytest.mark.parametrize("causal", [False, True])
def test_split_tile_order_full_sequence_accuracy(causal):
    """The full-sequence split-tile order (every row, two 64-key streams merged) against fp64 attention: as accurate as
    the reference's order (<= 1.10 x its mean error, no more bad elements), with and without the causal mask."""
    inp = oracle.Inputs(1, 4, 512, 700, causal=causal)
    ref = oracle.check_fp64(inp, oracle.emulate(inp, rows=0), rows=512)
    st = oracle.check_fp64(inp, oracle.emulate(inp, rows=0, split_tiles=True), rows=512)
    assert st["bad"] <= ref["bad"] and st["mean_err"] <= 1.10 * ref["mean_err"], (st, ref)


def test_split_tile_order_duplicated_halves():
    """Keys 64..127 of every tile made copies of keys 0..63: the two streams then see the same scores, take the same
    rebases and merge with scale 1, which doubles O and l; the output equals the reference's order (one stream over
    the same 128 keys, same maxima, same P) up to the fp32 accumulation order of O and l."""
    B, H, S, SK = 1, 2, 64, 1024
    inp = oracle.Inputs(B, H, S, SK)
    k = inp.k.reshape(B, SK // 128, 128, H, D)
    v = inp.v.reshape(B, SK // 128, 128, H, D)
    ks = inp.ks[: B * SK * H * 4].reshape(B, SK // 128, 128, H, 4)
    k[:, :, 64:] = k[:, :, :64]
    v[:, :, 64:] = v[:, :, :64]
    ks[:, :, 64:] = ks[:, :, :64]
    ref = oracle.bf16_to_f32(oracle.emulate(inp, splits=2, rows=0)).astype(np.float64)
    st = oracle.bf16_to_f32(oracle.emulate(inp, splits=2, rows=0, split_tiles=True)).astype(np.float64)
    # one bf16 rounding step (2^-8 relative) at most
    assert np.all(np.abs(st - ref) <= np.abs(ref) * 2.0 ** -8 + 1e-6)
    assert np.mean(st == ref) > 0.9


@pytest.mark.parametrize("boost", [0, 3])
def test_split_tile_order_accuracy(boost):
    """Against fp64 attention the split-tile order is as accurate as the reference's (its bar: <= 1.10 x the mean error,
    no more bad elements). boost = 3 raises the K scales of keys 64..127 of every tile by 3 binades (scores x 8), so
    the two streams rebase to very different biases and the merge's scaling of one stream by 2^(512 (b_min - b))
    decides the result: a merge that scaled the wrong stream, or by the inverse factor, fails this."""
    B, H, S, SK = 1, 4, 128, 2048
    inp = oracle.Inputs(B, H, S, SK)
    if boost:
        ks = inp.ks[: B * SK * H * 4].reshape(B, SK // 128, 128, H, 4)
        ks[:, :, 64:] += boost
    ref_stats = oracle.check_fp64(inp, oracle.emulate(inp, splits=4, rows=0), rows=S)
    st_stats = oracle.check_fp64(inp, oracle.emulate(inp, splits=4, rows=0, split_tiles=True), rows=S)
    assert st_stats["bad"] <= ref_stats["bad"]
    assert st_stats["mean_err"] <= 1.10 * ref_stats["mean_err"]


def _scale_for_c(c_target):
    """An f32 softmax scale whose f32(scale * log2 e) is exactly c_target (searched among neighbouring f32 values)."""
    l2e = np.float32(1.4426950408889634)
    s = np.float32(c_target) / l2e
    for _ in range(64):
        c = np.float32(s) * l2e
        if c == np.float32(c_target):
            return float(s)
        s = np.nextafter(s, np.float32(np.inf) if c < c_target else np.float32(0), dtype=np.float32)
    raise AssertionError("no f32 scale found")


@pytest.mark.parametrize("splits", [0, 2])
def test_qk_scale_power_of_two_is_a_q_exponent_shift(splits):
    """The in-kernel softmax scale (extension) with c = scale log2 e = 2^-3 exactly (mantissa 1) must give the same bits
    as the unscaled recipe on Q scales lowered by 3 binades: the exponent goes into the Q E8M0 bytes, nothing else."""
    B, H, S, SK = 1, 2, 64, 700
    scaled = oracle.Inputs(B, H, S, SK, qk_scale=_scale_for_c(0.125))
    shifted = oracle.Inputs(B, H, S, SK)
    n = B * S * H * 4
    assert (shifted.qs[:n] >= 3 + 9).all()
    shifted.qs[:n] -= 3
    np.testing.assert_array_equal(oracle.emulate(scaled, splits=splits, rows=0), oracle.emulate(shifted, splits=splits, rows=0))


@pytest.mark.parametrize("splits", [0, 4])
def test_qk_scale_mantissa(splits):
    """c = 1.5 x 2^-3 (mantissa 1.5): the recipe multiplies S by 1.5 after seeding it with b / 1.5. Against fp64
    attention with scores ln2 c q.k it must stay as accurate as the unscaled recipe (a missing or inverted mantissa
    multiply changes every score by 1.5x and fails), and the CPU fp32 attention must agree with the fp64 check."""
    B, H, S, SK = 1, 2, 64, 1500
    base = oracle.Inputs(B, H, S, SK)
    ref = oracle.check_fp64(base, oracle.emulate(base, splits=splits, rows=0), rows=S)
    inp = oracle.Inputs(B, H, S, SK, qk_scale=_scale_for_c(0.1875))
    got = oracle.check_fp64(inp, oracle.emulate(inp, splits=splits, rows=0), rows=S)
    assert got["bad"] == 0 and got["mean_err"] <= 2.0 * ref["mean_err"], (got, ref)
    # the unscaled recipe on the same Q misses the factor 1.5 x 2^-3: far off
    wrong = oracle.check_fp64(inp, oracle.emulate(base, splits=splits, rows=0), rows=S)
    assert wrong["mean_err"] > 10 * got["mean_err"]
    _, f32 = oracle.attention_fp32(inp, rows=S)
    u = np.ascontiguousarray(f32, dtype=np.float32).view(np.uint32)
    as_bf16 = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)   # round to nearest even
    assert oracle.check_fp64(inp, as_bf16, rows=S)["mean_err"] < 0.5 * got["mean_err"]


def test_generator_matches_reference_harness():
    """The oracle's input generator is byte-identical to the reference harness's own (tests/gpu/ref_host.cpp:183-263),
    in all three data modes (lcg palette, uniform bytes, normal MXFP8) and on every shape of run_ref.sh:57, the
    determinism list and the BASELINE configs: tests/golden/ref_inputs.json holds the SHA-256 of each buffer that the
    reference's harness, built from its source, dumped (tests/golden/make_ref_inputs_fixture.py)."""
    import hashlib
    import json
    with open(os.path.join(os.path.dirname(__file__), "golden", "ref_inputs.json")) as f:
        fx = json.load(f)
    assert len(fx["entries"]) >= 50
    for e in fx["entries"]:
        inp = oracle.Inputs(e["B"], e["H"], e["S"], e["SK"], HK=e["H"] // e["gqa"], mode=e["mode"])
        for ext, arr in (("q", inp.q), ("k", inp.k), ("v", inp.v), ("qs", inp.qs), ("ks", inp.ks)):
            want = e["digests"][ext]
            data = np.ascontiguousarray(arr).tobytes()
            assert len(data) == want["bytes"], (e, ext)
            assert hashlib.sha256(data).hexdigest() == want["sha256"], (e["B"], e["H"], e["S"], e["SK"], e["mode"], ext)
