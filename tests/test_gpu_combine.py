"""The two combine kernels on the same partial rows, launched directly through the C ABI.

fmha_fwd_hd128_mxfp8_v3_kvsplit_combine8h merges each row's splits in order; the extension
fmha_fwd_hd128_mxfp8_v3_kvsplit_combine_wide spreads them over a block's 4 waves (a quarter each, ceil(splits / 4)
splits) and merges the quarters in order. With at most 4 splits every quarter holds one split, and the quarter merge
performs the same operations as the in-order merge (a single split's state is (lse, 1, x)), so the two kernels must
agree bit for bit; with more splits only the rounding order differs. Both are also checked against the oracle's
combine (epilogue.rs:89-167) within the exp2 approximation. Ragged row counts exercise the tail groups."""
import ctypes

import numpy as np
import pytest

import oracle
from amdgpu_rustdsl_amd import lib

pytestmark = pytest.mark.gpu
D = 128


def _run(kernel, ohat, lse, rows, splits, f32, device):
    import torch
    oh = torch.from_numpy(np.ascontiguousarray(ohat)).to(device)
    ls = torch.from_numpy(np.ascontiguousarray(lse, np.float32)).to(device)
    out = torch.full((rows, D), float("nan"), dtype=torch.bfloat16, device=device)
    a = lib.CombineArgs()
    a.ptr_ohat, a.ptr_lse, a.ptr_out = oh.data_ptr(), ls.data_ptr(), out.data_ptr()
    a.rows_total, a.d, a.splits = rows, D, splits | (lib.KVS_F32_PARTIALS if f32 else 0)
    st = torch.cuda.current_stream(device).cuda_stream
    if kernel == "8h":
        rc = lib.raw.fmha_mxfp8_launch_combine(ctypes.byref(a), (rows * 16 + 255) // 256, st)
    else:
        rc = lib.raw.fmha_mxfp8_launch_combine_wide(ctypes.byref(a), (rows * 16 + 63) // 64, st)
    assert rc == 0
    torch.cuda.synchronize()
    return out.view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)


def _partials(rows, splits, f32, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((splits, rows, D)).astype(np.float32)
    lse = (rng.standard_normal((splits, rows)) * 4.0).astype(np.float32)
    lse[rng.random((splits, rows)) < 0.05] = -1.0e30   # empty ranges: weight 0
    ohat = x if f32 else x.astype(np.float16).view(np.uint16)
    return ohat, lse


@pytest.mark.parametrize("splits", [1, 2, 3, 4, 5, 8, 16, 32, 64])
@pytest.mark.parametrize("f32", [False, True], ids=["fp16", "f32"])
def test_combine_wide_against_combine8h(gpu, splits, f32):
    rows = 1000 + splits   # ragged: the last block's tail groups redo the last group
    print(f"[case] combine splits={splits} f32={f32} rows={rows}", flush=True)
    ohat, lse = _partials(rows, splits, f32, seed=100 + splits)
    o8 = _run("8h", ohat, lse, rows, splits, f32, gpu)
    ow = _run("wide", ohat, lse, rows, splits, f32, gpu)
    ref = oracle.combine(ohat, lse, rows, splits)
    assert not np.isnan(oracle.bf16_to_f32(ow)).any() and not np.isnan(oracle.bf16_to_f32(o8)).any()
    if splits <= 4:
        np.testing.assert_array_equal(ow, o8)
    fw, f8, fr = (oracle.bf16_to_f32(v).astype(np.float64) for v in (ow, o8, ref))
    # one bf16 rounding of a value of magnitude up to ~4 (the exp2 approximations move the weights by ~1e-7)
    tol = 2.0 ** -7 * np.maximum(np.abs(fr), 1.0)
    assert (np.abs(fw - fr) <= tol).all(), float(np.abs(fw - fr).max())
    assert (np.abs(f8 - fr) <= tol).all(), float(np.abs(f8 - fr).max())
