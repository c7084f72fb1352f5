"""Helpers of the GPU parity tests: upload the oracle's seeded inputs and run the op through the C ABI."""
import numpy as np
import torch

import oracle
from amdgpu_rustdsl_amd import lib, ops

D = 128


def upload(inp, device):
    """Device tensors of an oracle.Inputs (descale tensors viewed from allocations with the zeroed slack)."""
    B, H, HK, S, SK = inp.B, inp.H, inp.HK, inp.S, inp.SK
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)
    q = t(inp.q).view(B, S, H, D)
    k = t(inp.k).view(B, SK, HK, D)
    v = t(inp.v).view(B, SK, HK, D)
    qs_all = t(inp.qs)
    ks_all = t(inp.ks)
    qs = qs_all[: B * S * H * 4].view(B, S, H, 4)
    ks = ks_all[: B * SK * HK * 4].view(B, SK, HK, 4)
    if inp.vs32 is not None:   # extension: per-32-key V scales [B, ceil(SK/32), HK, 128]
        vs = t(inp.vs32).view(B, (SK + 31) // 32, HK, D)
    else:
        vs = t(inp.vd_buf)
    return q, k, v, qs, ks, vs


def chunks(inp, path="auto", splits=None):
    """The reference's KV-split chunk count for a run of `path` (0 when the run is not a KV split): the forced count,
    or the dispatch's."""
    if path == "kvsplit":
        return splits or 4
    if path == "auto" and not inp.causal:
        p, sp = lib.select_path(inp.B, inp.H, inp.S, inp.SK)
        return sp if p == "kvsplit" else 0
    return 0


def run(inp, device, path="auto", splits=None, lse=False, poison=True, partials="fp16", causal_pair="auto", kv_fill=True):
    """Runs the op; returns (bf16 output as uint16 numpy [B*S*H*128], (path, splits), lse tensor or None)."""
    q, k, v, qs, ks, vs = upload(inp, device)
    out = torch.empty(inp.B, inp.S, inp.H, D, dtype=torch.bfloat16, device=device)
    if poison:
        out.view(torch.int16).fill_(0x7fc1)   # NaN: every element must be written
    lse_t = torch.full((inp.B, inp.H, inp.S), float("nan"), dtype=torch.float32, device=device) if lse else None
    used = ops.fmha_fwd_mxfp8(q, k, v, qs, ks, vs, out, path=path, splits=splits, lse=lse_t, causal=inp.causal,
                              partials=partials, softmax_scale=inp.qk_scale if inp.qk_scale > 0 else None,
                              causal_pair=causal_pair, kv_fill=kv_fill)
    torch.cuda.synchronize()
    o = out.view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)
    return o, used, lse_t


def compare_to_emulation(out, emu, inp, rows):
    """Element statistics of the GPU output against the recipe emulation on `rows` of every (b,h): the first n rows,
    or a list of rows."""
    sel = oracle.row_list(inp.S, rows)
    o = out.reshape(inp.B, inp.S, inp.H, D)[:, sel]
    e = emu.reshape(inp.B, inp.S, inp.H, D)[:, sel]
    of = oracle.bf16_to_f32(o).astype(np.float64)
    ef = oracle.bf16_to_f32(e).astype(np.float64)
    diff = np.abs(of - ef)
    return {"exact": float(np.mean(o == e)), "max_abs": float(np.nanmax(diff)) if diff.size else 0.0,
            "mean_abs": float(np.mean(diff)), "nan": int(np.isnan(of).sum())}


def lse_reference(inp, rows):
    """float64 natural-log LSE [B, H, rows] of the dequantised inputs (scores ln2 c q.k, the kernels' base-2 convention,
    c the in-kernel softmax scale's multiplier or 1)."""
    dec = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy().astype(np.float64)
    dec[[0x7F, 0xFF]] = 0.0
    B, H, HK, S, SK = inp.B, inp.H, inp.HK, inp.S, inp.SK
    q = dec[inp.q].reshape(B, S, H, 4, 32) * 2.0 ** (inp.qs[: B * S * H * 4].reshape(B, S, H, 4, 1).astype(np.float64) - 127)
    k = dec[inp.k].reshape(B, SK, HK, 4, 32) * 2.0 ** (inp.ks[: B * SK * HK * 4].reshape(B, SK, HK, 4, 1).astype(np.float64) - 127)
    q, k = q.reshape(B, S, H, D), k.reshape(B, SK, HK, D)
    g = H // HK
    out = np.zeros((B, H, rows))
    for b in range(B):
        for h in range(H):
            s = q[b, :rows, h] @ k[b, :, h // g].T * (np.log(2.0) * score_scale(inp))
            if inp.causal:
                i = np.arange(rows)[:, None]
                t = np.arange(SK)[None, :]
                s = np.where(t <= i + SK - S, s, -np.inf)
            m = s.max(1, keepdims=True)
            out[b, h] = (m + np.log(np.exp(s - m).sum(1, keepdims=True)))[:, 0]
    return out


def run_direct(inp, device, kernel):
    """Launches one kernel through its C-ABI launcher (validate first), as a reference-style launcher does:
    kernel "vs128" (fmha_mxfp8_launch_vs128: the 256-row kernel, 512 threads, grid (ceil(S/256), H, B)), "t128"
    (fmha_mxfp8_launch_t128: the reference-named 128-row kernel with its 256 threads) or "t128_split_tiles". Returns the
    bf16 output as uint16 numpy [B*S*H*128] (NaN-poisoned before the launch)."""
    import ctypes
    import math
    from amdgpu_rustdsl_amd import lib
    q, k, v, qs, ks, vs = upload(inp, device)
    B, H, HK, S, SK = inp.B, inp.H, inp.HK, inp.S, inp.SK
    out = torch.empty(B, S, H, D, dtype=torch.bfloat16, device=device)
    out.view(torch.int16).fill_(0x7fc1)
    a = lib.fill_args(out.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), qs.data_ptr(), ks.data_ptr(), vs.data_ptr(),
                      B, H, HK, S, SK)
    a.flags = (lib.FLAG_CAUSAL if inp.causal else 0) | (lib.FLAG_V_SEQ32 if inp.vs32 is not None else 0)
    rows = 256 if kernel == "vs128" else 128
    grid = (math.ceil(S / rows), H, B)
    sz = lib.BufferSizes(ops._cap(q), ops._cap(k), ops._cap(v), ops._cap(out), ops._cap(qs), ops._cap(ks), ops._cap(vs), 0, 0)
    rc, msg = lib.validate("vs128" if kernel == "vs128" else "t128", a, sz, grid, HK=HK)
    assert rc == 0, msg
    fn = {"vs128": lib.raw.fmha_mxfp8_launch_vs128, "t128": lib.raw.fmha_mxfp8_launch_t128,
          "t128_split_tiles": lib.raw.fmha_mxfp8_launch_t128_split_tiles}[kernel]
    assert fn(ctypes.byref(a), *grid, torch.cuda.current_stream(device).cuda_stream) == 0
    torch.cuda.synchronize()
    return out.view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)


def _dequant(inp):
    """float64 dequantised Q [B,S,H,128], K and V [B,SK,HK,128], V with its scales as the oracle's float64 check takes
    them (mxfp8_oracle.c v_block_scale / v_tensor_descale): one E8M0 per 32 keys and column under per-32-key V scales,
    else the per-tensor descale."""
    dec = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy().astype(np.float64)
    dec[[0x7F, 0xFF]] = 0.0
    B, H, HK, S, SK = inp.B, inp.H, inp.HK, inp.S, inp.SK
    q = dec[inp.q].reshape(B, S, H, 4, 32) * 2.0 ** (inp.qs[: B * S * H * 4].reshape(B, S, H, 4, 1).astype(np.float64) - 127)
    k = dec[inp.k].reshape(B, SK, HK, 4, 32) * 2.0 ** (inp.ks[: B * SK * HK * 4].reshape(B, SK, HK, 4, 1).astype(np.float64) - 127)
    v = dec[inp.v[: B * SK * HK * D]].reshape(B, SK, HK, D)
    if inp.vs32 is not None:
        nb = (SK + 31) // 32
        e = np.asarray(inp.vs32, dtype=np.uint8)[: B * nb * HK * D].reshape(B, nb, HK, D).astype(np.float64)
        v = v * np.repeat(2.0 ** (e - 127), 32, axis=1)[:, :SK]
    else:
        v = v * float(inp.vdescale)
    return q.reshape(B, S, H, D), k.reshape(B, SK, HK, D), v


def score_scale(inp):
    """The base-2 score multiplier: 1, or under the in-kernel softmax scale c = f32(scale) * f32(log2 e) in f32
    (mxfp8_oracle.c qk_scaling_of)."""
    if not inp.qk_scale > 0:
        return 1.0
    return float(np.float32(inp.qk_scale) * np.float32(1.4426950408889634))


def fp64_rows(inp, rows):
    """float64 attention of the listed rows (base-2 scores, as ref_host.cpp:436-471 checks them; no causal mask) and,
    per row, the gap between its two largest scores and the sum of those two keys' score magnitudes sum_d |q_d k_d|
    (log2 units). Returns (out [B, n, H, 128], gap [B, n, H], mag [B, n, H])."""
    assert not inp.causal
    sel = oracle.row_list(inp.S, rows)
    q, k, v = _dequant(inp)
    B, H, HK = inp.B, inp.H, inp.HK
    g = H // HK
    out = np.zeros((B, sel.size, H, D))
    gap = np.zeros((B, sel.size, H))
    mag = np.zeros((B, sel.size, H))
    for b in range(B):
        for h in range(H):
            qs, ks = q[b, sel, h], k[b, :, h // g]
            s = (qs @ ks.T) * score_scale(inp)
            m = (np.abs(qs) @ np.abs(ks).T) * score_scale(inp)
            order = np.argsort(-s, axis=1)
            top = np.take_along_axis(s, order[:, :2], 1) if s.shape[1] > 1 else np.concatenate([s, s - np.inf], 1)
            gap[b, :, h] = top[:, 0] - top[:, 1]
            mag[b, :, h] = np.take_along_axis(m, order[:, :1], 1)[:, 0] + (
                np.take_along_axis(m, order[:, 1:2], 1)[:, 0] if s.shape[1] > 1 else 0.0)
            w = np.exp2(s - s.max(1, keepdims=True))
            out[b, :, h] = (w / w.sum(1, keepdims=True)) @ v[b, :, h // g]
    return out, gap, mag


def causal_rows(inp, rows):
    """float64 attention of the listed rows under the bottom-right causal mask (base-2 scores; a row with no visible
    key gives zeros), each row's visible-key count, and per element the largest change one e4m3 step of one key's P
    can make: max_k w_k 2^-3 |v_k,d - o_d| over the visible keys k (w_k the row's float64 softmax weights; 2^-3 is an
    e4m3 step relative to the value at the bottom of its binade). Returns (out [B, n, H, 128], vis [n],
    flip [B, n, H, 128])."""
    sel = oracle.row_list(inp.S, rows)
    q, k, v = _dequant(inp)
    B, H, HK, S, SK = inp.B, inp.H, inp.HK, inp.S, inp.SK
    g = H // HK
    vis = np.clip(sel.astype(np.int64) + SK - S + 1, 0, SK)
    out = np.zeros((B, sel.size, H, D))
    flip = np.zeros((B, sel.size, H, D))
    for b in range(B):
        for h in range(H):
            s = (q[b, sel, h] @ k[b, :, h // g].T) * score_scale(inp)
            s[np.arange(SK)[None, :] >= vis[:, None]] = -np.inf
            live = vis > 0
            s = s[live]
            w = np.exp2(s - s.max(1, keepdims=True))
            w /= w.sum(1, keepdims=True)
            vv = v[b, :, h // g]
            o = w @ vv
            out[b, live, h] = o
            # max over keys of w_k |v_k - o| per dim, in blocks of rows to bound the temporary
            f = np.zeros_like(o)
            for r0 in range(0, o.shape[0], 16):
                blk = w[r0:r0 + 16, :, None] * np.abs(vv[None, :, :] - o[r0:r0 + 16, None, :])
                f[r0:r0 + 16] = blk.max(1)
            flip[b, live, h] = f * 2.0 ** -3
    return out, vis, flip


def causal_bar(inp, out, emu, rows):
    """The causal bar against the oracle alone (no kernel output on the other side):
    - element-wise closeness to the recipe's emulation: within 0.05 on rows that see at least 64 keys (as without the
      mask), within 0.25 on rows with fewer, whose outputs rest on a few keys;
    - an element outside the harness tolerance (ref_host.cpp:466: |err| > 0.05 + 0.05 |ref|) that the emulation keeps
      inside it must differ from the emulation by no more than one e4m3 step of one key's P can move it (the MFMA's
      inexact sums can carry a P value across a rounding step), and such elements may lie in at most 2 % of the rows.
    Returns a dict of the figures (for the log) and the list of violations."""
    sel = oracle.row_list(inp.S, rows)
    ref, vis, flip = causal_rows(inp, rows)
    shape = (inp.B, inp.S, inp.H, D)
    o = oracle.bf16_to_f32(out.reshape(shape)[:, sel]).astype(np.float64)
    e = oracle.bf16_to_f32(emu.reshape(shape)[:, sel]).astype(np.float64)
    d = np.abs(o - e)
    many = vis >= 64
    tol = lambda x: np.abs(x - ref) <= 0.05 + 0.05 * np.abs(ref)
    extra = ~tol(o) & tol(e)
    explained = d <= 1.5 * flip + 2.0 ** -8 * np.abs(ref) + 1e-4
    rows_extra = int(extra.any(axis=3).sum())   # attention rows (b, query, h) holding such an element
    nrows = inp.B * sel.size * inp.H
    fig = {"max_abs_many": float(d[:, many].max()) if many.any() else 0.0,
           "max_abs_few": float(d[:, ~many].max()) if (~many).any() else 0.0,
           "bad_ours": int((~tol(o)).sum()), "bad_emulation": int((~tol(e)).sum()), "extra": int(extra.sum()),
           "extra_unexplained": int((extra & ~explained).sum()), "extra_rows": rows_extra, "rows": nrows}
    viol = []
    if fig["max_abs_many"] > 0.05:
        viol.append("max_abs over rows with >= 64 visible keys")
    if fig["max_abs_few"] > 0.25:
        viol.append("max_abs over rows with < 64 visible keys")
    if fig["extra_unexplained"]:
        viol.append("elements outside the tolerance beyond one P step")
    if rows_extra > 0.02 * nrows + 1:
        viol.append("too many rows with extra elements outside the tolerance")
    return fig, viol
