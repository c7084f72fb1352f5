"""GPU parity of the on-GPU MXFP8 quantisers (include/mxfp8_quant.h) against the oracle's restatement of the
reference generator's rule (ref_host.cpp:239-251), through the C ABI. Integer/byte work: bit-exact.

Inputs cover every finite and non-finite bf16 bit pattern, ragged row counts (a partial last workgroup), ragged
sequence blocks, an all-zero tensor, signed zeros, and end-to-end use as the FMHA's inputs.
"""
import math

import numpy as np
import pytest
import torch

import oracle
from amdgpu_rustdsl_amd import lib, ops

pytestmark = pytest.mark.gpu
D = 128


def _bf16_bits(a):
    return (np.asarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def _dev(bits, gpu):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(gpu).view(torch.bfloat16)


def _host(t):
    return t.cpu().numpy().reshape(-1)


def _all_patterns(seed):
    """Every 16-bit pattern once, shuffled into rows of 128 (blocks mix magnitudes, NaN, Inf, +-0, subnormals)."""
    p = np.arange(65536, dtype=np.uint16)
    np.random.default_rng(seed).shuffle(p)
    return p


def _rows_case(bits, mul, gpu):
    rows = bits.size // D
    x = _dev(bits, gpu).view(rows, D)
    sc = torch.full((rows, 4), 0xAB, dtype=torch.uint8, device=gpu)
    q = ops.quantize_mxfp8(x, sc, mul=mul)
    torch.cuda.synchronize()
    q_ref, s_ref = oracle.quant_rows_bf16(bits, mul)
    return _host(q), _host(sc), q_ref, s_ref


@pytest.mark.parametrize("mul", [1.0, 1.4426950408889634 / math.sqrt(128)])
def test_rows_every_bf16_pattern(gpu, mul):
    q, s, q_ref, s_ref = _rows_case(_all_patterns(1), mul, gpu)
    assert np.array_equal(s, s_ref), f"scales differ at {np.flatnonzero(s != s_ref)[:8]}"
    bad = np.flatnonzero(q != q_ref)
    assert bad.size == 0, f"{bad.size} bytes differ, first {bad[:8]}: gpu {q[bad[:8]]} oracle {q_ref[bad[:8]]}"


@pytest.mark.parametrize("rows", [1, 15, 17, 1000, 65536 + 7])
def test_rows_normal_ragged(gpu, rows):
    x = np.random.default_rng(rows).standard_normal(rows * D).astype(np.float32) * 3.0
    q, s, q_ref, s_ref = _rows_case(_bf16_bits(x), 1.0, gpu)
    assert np.array_equal(s, s_ref)
    assert np.array_equal(q, q_ref)


def test_rows_signed_zero_and_saturation(gpu):
    # -0 encodes as +0 (the generator's sign byte is x < 0); block maxima in (448, 512) 2^k saturate to 448
    x = np.zeros((4, D), np.float32)
    x[0, :] = -0.0
    x[1, :32] = np.linspace(-500.0, 500.0, 32)
    x[2, 32:64] = 1e-30
    x[3, :] = np.float32(-1e-3)
    q, s, q_ref, s_ref = _rows_case(_bf16_bits(x), 1.0, gpu)
    assert np.array_equal(s, s_ref) and np.array_equal(q, q_ref)
    assert (q[:D] == 0).all()


@pytest.mark.parametrize("n", [8, 4096 * 128, 3 * 2048 * 8 * 128 + 8])
def test_tensor_matches_oracle(gpu, n):
    x = np.random.default_rng(n).standard_normal(n).astype(np.float32)
    x[n // 3] = 37.5   # an outlier sets the descale
    bits = _bf16_bits(x)
    q, vs = ops.quantize_v(_dev(bits, gpu))
    torch.cuda.synchronize()
    q_ref, d_ref = oracle.quant_tensor_bf16(bits)
    assert vs[0].item() == d_ref
    assert np.array_equal(_host(q), q_ref)


def test_tensor_every_pattern_finite(gpu):
    bits = _all_patterns(2)
    f = oracle.bf16_to_f32(bits)
    bits = bits[np.isfinite(f)][: (np.isfinite(f).sum() // 8) * 8]
    q, vs = ops.quantize_v(_dev(bits, gpu))
    torch.cuda.synchronize()
    q_ref, d_ref = oracle.quant_tensor_bf16(bits)
    assert vs[0].item() == d_ref
    assert np.array_equal(_host(q), q_ref)


def test_tensor_many_divisors(gpu):
    """The quotient x / d (d = amax / 448) over many divisors: for each chosen maximum, every finite bf16 pattern at or
    below it. Covers the fast quotient path and the full-division path (tiny and huge d, subnormal x and quotients)."""
    pats = np.arange(65536, dtype=np.uint16)
    f = oracle.bf16_to_f32(pats)
    fin = pats[np.isfinite(f)]
    amaxes = [2.0 ** e for e in (-133, -126, -100, -97, -96, -60, -8, 0, 9, 40, 96, 97, 127)]
    amaxes += [np.float32(1.9921875) * 2.0 ** e for e in (-130, -96, -10, 0, 3, 95, 126)]   # all-ones bf16 mantissa
    for am in amaxes:
        a = np.float32(am)
        keep = fin[np.abs(oracle.bf16_to_f32(fin)) <= a]
        keep = np.concatenate([keep, _bf16_bits([a])])
        keep = np.concatenate([keep, np.zeros((-keep.size) % 8, np.uint16)])
        q, vs = ops.quantize_v(_dev(keep, gpu))
        torch.cuda.synchronize()
        q_ref, d_ref = oracle.quant_tensor_bf16(keep)
        assert vs[0].item() == d_ref, f"amax {am}"
        bad = np.flatnonzero(_host(q) != q_ref)
        assert bad.size == 0, f"amax {am}: {bad.size} bytes differ"


def test_tensor_all_zero(gpu):
    q, vs = ops.quantize_v(torch.zeros(64, D, dtype=torch.bfloat16, device=gpu))
    torch.cuda.synchronize()
    q_ref, d_ref = oracle.quant_tensor_bf16(np.zeros(64 * D, np.uint16))
    assert vs[0].item() == d_ref == 0.0
    assert np.array_equal(_host(q), q_ref)


def test_tensor_repeat_reuses_scale_buffer(gpu):
    # every call rewrites the partial maxima it reads: a second, smaller tensor gets its own descale
    big = torch.randn(256, D, device=gpu, dtype=torch.bfloat16) * 10
    small = torch.randn(64, D, device=gpu, dtype=torch.bfloat16)
    q = torch.empty(256 * D, dtype=torch.uint8, device=gpu)
    vs = torch.zeros(1024, dtype=torch.float32, device=gpu)
    for x in (big, small):
        lib.quantize_tensor(x.data_ptr(), q.data_ptr(), vs.data_ptr(), x.numel(), x.numel() * 2, q.numel(), 4096,
                            torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        bits = x.view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)
        q_ref, d_ref = oracle.quant_tensor_bf16(bits)
        assert vs[0].item() == d_ref
        assert np.array_equal(q[: x.numel()].cpu().numpy(), q_ref)


@pytest.mark.parametrize("B,SK,HK", [(1, 32, 1), (2, 100, 3), (1, 2048, 8), (3, 1, 2)])
def test_seq32_matches_oracle(gpu, B, SK, HK):
    x = np.random.default_rng(SK).standard_normal(B * SK * HK * D).astype(np.float32)
    x *= np.exp(np.random.default_rng(7).uniform(-20, 20, x.size)).astype(np.float32)   # wide exponent range
    bits = _bf16_bits(x)
    q, sc = ops.quantize_v_seq32(_dev(bits, gpu).view(B, SK, HK, D))
    torch.cuda.synchronize()
    q_ref, s_ref = oracle.quant_seq32_bf16(bits, B, SK, HK)
    assert np.array_equal(_host(sc), s_ref)
    assert np.array_equal(_host(q), q_ref)


def test_rejections(gpu):
    x = torch.zeros(16, D, dtype=torch.bfloat16, device=gpu)
    q = torch.empty(16 * D, dtype=torch.uint8, device=gpu)
    s = torch.empty(64, dtype=torch.uint8, device=gpu)
    st = torch.cuda.current_stream().cuda_stream
    with pytest.raises(lib.FmhaError, match="GV-HOST-EXTENT"):
        lib.quantize_rows(x.data_ptr(), q.data_ptr(), s.data_ptr(), 16, 1.0, x.numel() * 2, q.numel(), 63, st)
    with pytest.raises(lib.FmhaError, match="alignment"):
        lib.quantize_rows(x.data_ptr() + 2, q.data_ptr(), s.data_ptr(), 15, 1.0, 4096, 4096, 64, st)
    with pytest.raises(lib.FmhaError, match="multiple of 8"):
        lib.quantize_tensor(x.data_ptr(), q.data_ptr(), s.data_ptr(), 12, 4096, 4096, 64, st)
    with pytest.raises(lib.FmhaError, match="GV-HOST-EXTENT"):
        lib.quantize_tensor(x.data_ptr(), q.data_ptr(), s.data_ptr(), 16 * D, 4096, 4096, 4095, st)


def test_fmha_from_bf16_uses_the_quantised_inputs(gpu):
    """fmha_fwd_bf16_via_mxfp8 == fmha_fwd_mxfp8 on the oracle-quantised bytes (bit-identical output), and both are
    within the MXFP8 error of fp32 attention on the bf16 inputs."""
    B, H, S, SK = 1, 4, 512, 640
    g = torch.Generator(device=gpu)
    g.manual_seed(3)
    qf, kf, vf = (torch.randn(B, n, H, D, generator=g, device=gpu, dtype=torch.bfloat16) for n in (S, SK, SK))
    out = ops.fmha_fwd_bf16_via_mxfp8(qf, kf, vf)
    bits = lambda t: t.view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)
    q8, qs8 = oracle.quant_rows_bf16(bits(qf), 1.4426950408889634 / math.sqrt(D))
    k8, ks8 = oracle.quant_rows_bf16(bits(kf))
    v8, vd = oracle.quant_tensor_bf16(bits(vf))
    up = lambda a, *shape: torch.from_numpy(a).to(gpu).view(*shape)
    qs = ops.alloc_scales(B, S, H, gpu)
    ks = ops.alloc_scales(B, SK, H, gpu)
    qs.copy_(up(qs8, B, S, H, 4))
    ks.copy_(up(ks8, B, SK, H, 4))
    vs = torch.zeros(1024, dtype=torch.float32, device=gpu)
    vs[0] = float(vd)
    ref = torch.empty_like(out)
    ops.fmha_fwd_mxfp8(up(q8, B, S, H, D), up(k8, B, SK, H, D), up(v8, B, SK, H, D), qs, ks, vs, ref)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    att = torch.softmax(torch.einsum("bshd,bthd->bhst", qf.float(), kf.float()) / math.sqrt(D), dim=-1)
    exact = torch.einsum("bhst,bthd->bshd", att, vf.float())
    err = (out.float() - exact).abs()
    assert err.mean().item() < 0.01 and err.max().item() < 0.1


def test_fmha_from_bf16_with_v_seq32(gpu):
    """Extension end to end: bf16 -> on-GPU quantisers with per-32-key V scales -> FMHA reading them. Equals the FMHA on
    the oracle-quantised bytes (bit-identical), and is within the MXFP8 error of fp32 attention on the bf16 inputs."""
    B, H, S, SK = 1, 4, 512, 650
    g = torch.Generator(device=gpu)
    g.manual_seed(4)
    qf, kf, vf = (torch.randn(B, n, H, D, generator=g, device=gpu, dtype=torch.bfloat16) for n in (S, SK, SK))
    out = ops.fmha_fwd_bf16_via_mxfp8(qf, kf, vf, v_scales="seq32")
    bits = lambda t: t.view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)
    q8, qs8 = oracle.quant_rows_bf16(bits(qf), 1.4426950408889634 / math.sqrt(D))
    k8, ks8 = oracle.quant_rows_bf16(bits(kf))
    v8, vs8 = oracle.quant_seq32_bf16(bits(vf), B, SK, H)
    up = lambda a, *shape: torch.from_numpy(a).to(gpu).view(*shape)
    qs = ops.alloc_scales(B, S, H, gpu)
    ks = ops.alloc_scales(B, SK, H, gpu)
    qs.copy_(up(qs8, B, S, H, 4))
    ks.copy_(up(ks8, B, SK, H, 4))
    ref = torch.empty_like(out)
    ops.fmha_fwd_mxfp8(up(q8, B, S, H, D), up(k8, B, SK, H, D), up(v8, B, SK, H, D), qs, ks,
                       up(vs8, B, (SK + 31) // 32, H, D), ref)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    att = torch.softmax(torch.einsum("bshd,bthd->bhst", qf.float(), kf.float()) / math.sqrt(D), dim=-1)
    exact = torch.einsum("bhst,bthd->bshd", att, vf.float())
    err = (out.float() - exact).abs()
    tensor_out = ops.fmha_fwd_bf16_via_mxfp8(qf, kf, vf)
    err_t = (tensor_out.float() - exact).abs()
    print(f"[case] bf16 via mxfp8: seq32 mean {err.mean().item():.3g} max {err.max().item():.3g}; "
          f"tensor mean {err_t.mean().item():.3g}", flush=True)
    assert err.mean().item() < 0.01 and err.max().item() < 0.1


@pytest.mark.parametrize("scale", [1.0 / math.sqrt(D), 0.05])
def test_fmha_from_bf16_scale_in_kernel(gpu, scale):
    """Extension end to end: Q quantised as it is and the softmax scale applied in the kernel
    (scale_in_kernel=True) against fp32 attention on the bf16 inputs, within the MXFP8 error bar of the reference's
    convention (Q quantised with the scale folded in) on the same inputs."""
    B, H, S, SK = 1, 4, 512, 640
    g = torch.Generator(device=gpu)
    g.manual_seed(5)
    qf, kf, vf = (torch.randn(B, n, H, D, generator=g, device=gpu, dtype=torch.bfloat16) for n in (S, SK, SK))
    att = torch.softmax(torch.einsum("bshd,bthd->bhst", qf.float(), kf.float()) * scale, dim=-1)
    exact = torch.einsum("bhst,bthd->bshd", att, vf.float())
    folded = ops.fmha_fwd_bf16_via_mxfp8(qf, kf, vf, softmax_scale=scale)
    inkernel = ops.fmha_fwd_bf16_via_mxfp8(qf, kf, vf, softmax_scale=scale, scale_in_kernel=True)
    torch.cuda.synchronize()
    e_fold = (folded.float() - exact).abs()
    e_in = (inkernel.float() - exact).abs()
    print(f"[case] scale {scale}: folded mean {e_fold.mean().item():.3e} max {e_fold.max().item():.3e}; "
          f"in kernel mean {e_in.mean().item():.3e} max {e_in.max().item():.3e}", flush=True)
    assert e_in.mean().item() <= 1.25 * e_fold.mean().item() and e_in.max().item() < 0.1
