"""The allocation-free entry fmha_fwd_hd128_mxfp8_auto_noalloc (include/fmha_mxfp8.h) against the one-call entry
fmha_fwd_hd128_mxfp8_auto with a caller's workspace: the same kernels on the same inputs, so the outputs must be
bit-identical. Two KV-split calls in a row, the second on a smaller shape (the library's scratch keeps the first
call's partials), then a full-sequence call and the size limit."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from amdgpu_rustdsl_amd import lib, ops
from tests import gpu_util

pytestmark = pytest.mark.gpu


def _params(inp, tensors, out, path=-1, splits=0):
    q, k, v, qs, ks, vs = tensors
    p = lib.Params()
    p.o, p.q, p.k, p.v = out.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr()
    p.q_descale, p.k_descale, p.v_descale, p.lse = qs.data_ptr(), ks.data_ptr(), vs.data_ptr(), None
    p.bytes_q, p.bytes_k, p.bytes_v, p.bytes_o = ops._cap(q), ops._cap(k), ops._cap(v), ops._cap(out)
    p.bytes_q_descale, p.bytes_k_descale, p.bytes_v_descale = ops._cap(qs), ops._cap(ks), ops._cap(vs)
    p.B, p.H, p.HK, p.S, p.SK = inp.B, inp.H, inp.HK, inp.S, inp.SK
    p.path, p.splits = path, splits
    return p


def _both(gpu, inp, path=-1, splits=0):
    tensors = gpu_util.upload(inp, gpu)
    st = torch.cuda.current_stream(gpu).cuda_stream
    out_ref = torch.full((inp.B, inp.S, inp.H, 128), float("nan"), dtype=torch.bfloat16, device=gpu)
    out_na = torch.full_like(out_ref, float("nan"))
    p = _params(inp, tensors, out_ref, path, splits)
    used = lib.select_path(inp.B, inp.H, inp.S, inp.SK) if path < 0 else (lib.PATH_NAMES[path], splits)
    # (sized for the partials of the chunk fill, as the scratch array holds them: both entries then run the same)
    parts = lib.kv_partials(inp.B, inp.H, inp.S, inp.SK, used[1]) if used[0] == "kvsplit" else 0
    ws_bytes = lib.workspace_bytes(inp.B, inp.H, inp.S, parts) if used[0] == "kvsplit" else 0
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=gpu)
    got_ref = lib.run_auto(p, ws.data_ptr(), ws_bytes, st)
    p.o = out_na.data_ptr()
    got_na = lib.run_auto_noalloc(p, st)
    torch.cuda.synchronize()
    assert got_ref == got_na and got_ref.partials == got_na.partials
    a = out_ref.view(torch.int16).cpu().numpy()
    b = out_na.view(torch.int16).cpu().numpy()
    return got_na, a, b


def test_noalloc_matches_workspace_entry(gpu):
    cases = [
        ("cfg5_B1H8S128_SK16384_split8", oracle.Inputs(1, 8, 128, 16384), lib.PATH_KVSPLIT, 8),
        ("smaller_B1H4S128_SK4096_split2", oracle.Inputs(1, 4, 128, 4096, seed_mix=7), lib.PATH_KVSPLIT, 2),
        ("auto_split4_B1H8S512_SK4096", oracle.Inputs(1, 8, 512, 4096, seed_mix=3), -1, 0),
        ("full_sequence_B2H8S1024", oracle.Inputs(2, 8, 1024, 1024, seed_mix=5), -1, 0),
    ]
    for name, inp, path, splits in cases:
        print(f"[case] noalloc {name}", flush=True)
        used, a, b = _both(gpu, inp, path, splits)
        print(f"[case] noalloc {name} path={used}", flush=True)
        assert not np.isnan(oracle.bf16_to_f32(b.view(np.uint16))).any()
        assert np.array_equal(a, b), f"{name}: {np.mean(a != b):.3g} of the elements differ"


def test_noalloc_allocates_nothing(gpu):
    """After a first call (which looks the scratch array up and loads the code objects), calls of the allocation-free
    entry leave the device's free memory unchanged: no hipMalloc, no allocating library routine."""
    inp = oracle.Inputs(1, 8, 128, 16384)
    tensors = gpu_util.upload(inp, gpu)
    st = torch.cuda.current_stream(gpu).cuda_stream
    out = torch.empty((inp.B, inp.S, inp.H, 128), dtype=torch.bfloat16, device=gpu)
    p = _params(inp, tensors, out, lib.PATH_KVSPLIT, 8)
    lib.run_auto_noalloc(p, st)
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info(gpu)
    for _ in range(20):
        lib.run_auto_noalloc(p, st)
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info(gpu)
    assert free1 == free0, f"device free memory changed by {free0 - free1} bytes over 20 calls"


def test_noalloc_rejects_bad_split_count(gpu):
    """An invalid forced split count gets the entry's own error (GV-HOST-PATH), not the scratch-size one."""
    p = lib.Params()
    p.B, p.H, p.HK, p.S, p.SK, p.path, p.splits = 1, 8, 8, 128, 16384, lib.PATH_KVSPLIT, 16
    err = ctypes.create_string_buffer(256)
    po, so = ctypes.c_int(-1), ctypes.c_int(-1)
    rc = lib.raw.fmha_fwd_hd128_mxfp8_auto_noalloc(ctypes.byref(p), None, ctypes.byref(po), ctypes.byref(so), err, 256)
    assert rc == lib.FMHA_ERR_PATH and b"GV-HOST-PATH" in err.value


def test_noalloc_rejects_oversized_split(gpu):
    """A split whose workspace exceeds the scratch array is refused before any GPU work."""
    p = lib.Params()
    p.B, p.H, p.HK, p.S, p.SK, p.path, p.splits = 1, 8, 8, 2048, 2048, lib.PATH_KVSPLIT, 8
    err = ctypes.create_string_buffer(256)
    po, so = ctypes.c_int(-1), ctypes.c_int(-1)
    rc = lib.raw.fmha_fwd_hd128_mxfp8_auto_noalloc(ctypes.byref(p), None, ctypes.byref(po), ctypes.byref(so), err, 256)
    assert rc == lib.FMHA_ERR_WORKSPACE and b"GV-HOST-WORKSPACE" in err.value
