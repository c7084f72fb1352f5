"""The MXFP8 FMHA forward op on torch device tensors, mirroring the reference's ``fmha_fwd_mxfp8``
(python/amdgpu_jit/ops.py:88-143): same arguments, layouts, path names and errors, over the C ABI of
include/fmha_mxfp8.h (``amdgpu_rustdsl_amd.lib``). torch is used for device memory and the current stream only.
"""
import ctypes
import math

import torch

from . import lib

D = 128
FMHA_VS128 = "fmha_fwd_hd128_mxfp8_v3_vs128"
FMHA_T128 = "fmha_fwd_hd128_mxfp8_v3_t128"
FMHA_KVSPLIT = "fmha_fwd_hd128_mxfp8_v3_kvsplit"
FMHA_COMBINE = "fmha_fwd_hd128_mxfp8_v3_kvsplit_combine8h"


def select_path(B, H, S, SK):
    """(path, splits) of the shipped dispatch (``dispatch::mxfp8_prefill_path``, dispatch.rs:494-511)."""
    return lib.select_path(B, H, S, SK)


def _cap(t):
    """Bytes from the tensor's first element to the end of its storage (the allocation the kernel may touch)."""
    return t.untyped_storage().nbytes() - t.storage_offset() * t.element_size()


def _expect(t, name, shape, esize, align=1):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a torch tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name}: expected a device tensor, got {t.device}")
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name}: expected shape {tuple(shape)}, got {tuple(t.shape)}")
    if t.element_size() != esize:
        raise ValueError(f"{name}: expected {esize}-byte elements, got {t.element_size()}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: expected a contiguous tensor")
    if t.data_ptr() % align:
        raise ValueError(f"{name}: expected {align}-byte alignment")


_workspace = {}


def _ws(device, stream, nbytes):
    """Persistent KV-split workspace per (device, stream), grown on demand (ops.py:73-85), with the turn word of its
    slots (host memory, owned by this op: calls on one stream take the slots in turn)."""
    key = (device, stream)
    ent = _workspace.get(key)
    if ent is None or ent[0].numel() < nbytes:
        ent = _workspace[key] = (torch.empty(nbytes, dtype=torch.uint8, device=device), ctypes.c_uint32(0))
    return ent


def fmha_fwd_mxfp8(q, k, v, q_scale, k_scale, v_scale, out, *, path="auto", splits=None, specialize=True, stream=None, check=True,
                   lse=None, causal=False, partials="fp16", softmax_scale=None, causal_pair="auto", kv_fill=True):
    """Attention forward on MXFP8 inputs with head dim 128, written into ``out``; returns the (path, splits) that ran,
    splits being the KV split's chunk count as in the reference op (0 off the KV split). The returned tuple's
    ``.partials`` gives the partials per row that ran: the chunks times the blocks each chunk was spread over (the
    KV fill below).

    Scores are base-2: the kernels compute softmax2(q . k) over dequantised q and k, so a caller that wants the usual
    softmax(q k^T / sqrt(128)) multiplies q by log2(e) / sqrt(128) before quantising it (``fmha_fwd_bf16_via_mxfp8``
    does this). Tensors, all on one device, contiguous:
      q [B, S, H, 128] and k, v [B, SK, HK, 128]: e4m3 bytes (uint8 or float8_e4m3fn); H / HK is 1, 2, 4, 8 or 16.
      q_scale [B, S, H, 4], k_scale [B, SK, HK, 4]: one E8M0 byte per 32 elements of each row. The kernels read up to
        2048 H (q) and 2560 H (k) bytes past the end of these tensors, which must be zero: take them from
        ``alloc_scales``.
      v_scale: a float32 buffer of at least 4 KiB whose element 0 is V's descale; or, as an extension, uint8
        [B, ceil(SK/32), HK, 128] holding one E8M0 per 32 keys and column (from ``quantize_v_seq32``).
      out [B, S, H, 128] bf16.
    path: "auto" picks the kernel the way the reference's dispatch does; "vs128", "t128" or "kvsplit" force one
    (``splits``: 2, 4 or 8 for "kvsplit", default 4). ``stream``: a hipStream_t handle (default: torch's current
    stream). ``specialize`` is accepted for callers of the reference op; the kernels take every shape at run time,
    so there is nothing to specialise. ``check=False`` skips the host-side validate rules (buffer extents, strides,
    grid) before the launch; the op's own shape checks still run.
    Extensions: ``lse`` (float32 [B, H, S]) receives the natural-log log-sum-exp of each query row (vs128 / t128);
    ``causal`` masks key t from query i unless t <= i + SK - S; ``partials="fp32"`` keeps the KV split's partial rows
    in float32; ``softmax_scale`` makes the kernel apply scale * log2(e) to q . k itself (q then quantised unscaled);
    ``causal_pair`` ("auto", True, False): with ``causal``, one block runs query tiles x and T - 1 - x, so that every block
    has the same work; "auto" pairs when the unpaired grid exceeds the device's CUs (same output bits either way);
    ``kv_fill`` (default True): a KV split whose grid would leave CUs idle spreads each chunk's keys over up to 8
    blocks (``lib.kv_partials``), the combine merging every block's partial; False keeps the reference's one block
    per chunk. The fill changes the fp32 rounding order (each partial quantises P against its own running maximum),
    so its output bits differ from the reference grid's by a few ULP; which fill runs depends on the device's CU
    count.
    """
    pair_modes = {"auto": 0, True: 1, False: 2}
    if causal_pair not in pair_modes:
        raise ValueError(f"fmha_fwd_mxfp8: causal_pair must be 'auto', True or False, got {causal_pair!r}")
    if partials not in ("fp16", "fp32"):
        raise ValueError(f"fmha_fwd_mxfp8: partials must be 'fp16' or 'fp32', got {partials!r}")
    B, S, H, d = q.shape
    _, SK, HK, _ = k.shape
    if d != D or k.shape[3] != D or H % HK or (H // HK) & (H // HK - 1) or H // HK > 16:
        raise ValueError(f"fmha_fwd_mxfp8: head dim must be 128 and H a power-of-two multiple (<= 16) of HK (q {tuple(q.shape)}, k {tuple(k.shape)})")
    _expect(q, "q", (B, S, H, D), 1)
    _expect(k, "k", (B, SK, HK, D), 1)
    _expect(v, "v", (B, SK, HK, D), 1)
    _expect(q_scale, "q_scale", (B, S, H, 4), 1, align=4)
    _expect(k_scale, "k_scale", (B, SK, HK, 4), 1, align=4)
    _expect(out, "out", (B, S, H, D), 2)
    v_seq32 = v_scale.dtype == torch.uint8 and v_scale.dim() == 4
    if v_seq32:
        _expect(v_scale, "v_scale", (B, (SK + 31) // 32, HK, D), 1)
    elif _cap(v_scale) < 4:
        raise ValueError("v_scale: needs at least one f32")
    if lse is not None:
        _expect(lse, "lse", (B, H, S), 4)
    if path == "auto":
        path_id, nsplit = -1, 0
    elif path in ("vs128", "t128"):
        path_id, nsplit = lib.PATH_IDS[path], 0
    elif path == "kvsplit":
        path_id, nsplit = lib.PATH_KVSPLIT, splits or 4
        if nsplit not in (2, 4, 8):
            raise ValueError(f"fmha_fwd_mxfp8: unknown path {path!r} / splits {splits}")
    else:
        raise ValueError(f"fmha_fwd_mxfp8: unknown path {path!r} / splits {splits}")
    dev = q.device
    st = stream if stream is not None else torch.cuda.current_stream(dev).cuda_stream
    p = lib.Params()
    p.o, p.q, p.k, p.v = out.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr()
    p.q_descale, p.k_descale, p.v_descale = q_scale.data_ptr(), k_scale.data_ptr(), v_scale.data_ptr()
    p.lse = lse.data_ptr() if lse is not None else None
    p.bytes_q, p.bytes_k, p.bytes_v, p.bytes_o = _cap(q), _cap(k), _cap(v), _cap(out)
    p.bytes_q_descale, p.bytes_k_descale, p.bytes_v_descale = _cap(q_scale), _cap(k_scale), _cap(v_scale)
    p.B, p.H, p.HK, p.S, p.SK = B, H, HK, S, SK
    p.path, p.splits, p.causal = path_id, nsplit, int(bool(causal))
    p.f32_partials = int(partials == "fp32")
    p.v_seq32 = int(v_seq32)
    p.no_check = int(not check)
    p.causal_pair = pair_modes[causal_pair]
    p.kv_fill = 0 if kv_fill else 1
    if softmax_scale is not None:
        if not float(softmax_scale) > 0.0:
            raise ValueError(f"fmha_fwd_mxfp8: softmax_scale must be positive, got {softmax_scale!r}")
        p.softmax_scale = float(softmax_scale)
    # the workspace only matters for the KV split; size it for the split the dispatch will choose
    want_path, want_splits = (select_path(B, H, S, SK) if path_id < 0 else (path, nsplit))
    ws, ws_bytes = None, 0
    if want_path == "kvsplit" and not causal:
        # the entry's partials: the chunks, each spread over up to 8 blocks when the grid would leave CUs idle
        parts = lib.kv_partials(B, H, S, SK, want_splits) if kv_fill else want_splits
        ws_bytes = lib.workspace_bytes(B, H, S, parts)
        # room for the entry's workspace slots (consecutive calls then write partials the previous combine did not
        # just read), unless that would take more than 512 MiB
        slotted = lib.WORKSPACE_SLOTS * ((ws_bytes + 255) // 256 * 256)
        if slotted <= 512 << 20:
            ws_bytes = slotted
        buf, turn = _ws(dev, st, ws_bytes)
        ws = buf.data_ptr()
        p.ws_turn = ctypes.pointer(turn)
    with torch.cuda.device(dev):
        return lib.run_auto(p, ws, ws_bytes, st)


def alloc_scales(B, rows, H, device, fill=0):
    """An E8M0 scale tensor [B, rows, H, 4] viewed from an allocation with the zeroed slack tail of the kernel
    contract (512 H 4 bytes behind Q scales, 640 H 4 behind K scales: the larger is used for both)."""
    base = torch.zeros(B * rows * H * 4 + 640 * H * 4, dtype=torch.uint8, device=device)
    view = base[: B * rows * H * 4].view(B, rows, H, 4)
    if fill:
        view.fill_(fill)
    return view


def _bf16(x, name, rows=True):
    if not isinstance(x, torch.Tensor) or x.device.type != "cuda":
        raise ValueError(f"{name}: expected a device tensor")
    if rows and x.shape[-1] != D:
        raise ValueError(f"{name}: expected a last dimension of {D}, got {tuple(x.shape)}")
    return x.to(torch.bfloat16).contiguous()


def _stream(dev, stream):
    return stream if stream is not None else torch.cuda.current_stream(dev).cuda_stream


def quantize_mxfp8(x, scale_out, mul=1.0, stream=None):
    """On-GPU MXFP8 quantisation of rows x[..., 128] (bf16; other dtypes are cast to bf16 first) by the reference's
    generator rule (ref_host.cpp:239-247): per 32-element block E8M0 = clamp(floor(log2 amax) - 8 + 127, 0, 254) of
    the block of ``x * mul`` (f32), elements e4m3 round-to-nearest-even saturating at 448. Writes the scales into
    ``scale_out`` (uint8, shape x.shape[:-1] + (4,); ``alloc_scales`` gives one with the FMHA's zeroed slack) and
    returns the e4m3 bytes (uint8, shape of x). Runs fmha_mxfp8_quantize_rows (include/mxfp8_quant.h)."""
    xb = _bf16(x, "x")
    rows = xb.numel() // D
    _expect(scale_out, "scale_out", tuple(x.shape[:-1]) + (4,), 1, align=4)
    q = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    with torch.cuda.device(x.device):
        lib.quantize_rows(xb.data_ptr(), q.data_ptr(), scale_out.data_ptr(), rows, float(mul), _cap(xb), _cap(q), _cap(scale_out),
                          _stream(x.device, stream))
    return q


def quantize_v(x, stream=None):
    """On-GPU V quantisation with one f32 descale per tensor (ref_host.cpp:248-251): d = amax / 448, q = e4m3(x / d).
    Returns (q uint8 of x's shape, v_scale: a 4096-byte f32 buffer with d in element 0, the FMHA's V descale
    argument). x may have any shape whose element count is a multiple of 8. Runs fmha_mxfp8_quantize_tensor."""
    xb = _bf16(x, "x", rows=False)
    q = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    vs = torch.zeros(1024, dtype=torch.float32, device=x.device)
    with torch.cuda.device(x.device):
        lib.quantize_tensor(xb.data_ptr(), q.data_ptr(), vs.data_ptr(), xb.numel(), _cap(xb), _cap(q), _cap(vs), _stream(x.device, stream))
    return q, vs


def quantize_v_seq32(x, stream=None):
    """On-GPU V quantisation with one E8M0 per 32 keys along the sequence and per head_dim column (an extension; the
    reference's V scale is one f32 per tensor). x [B, SK, HK, 128] -> (q uint8 [B, SK, HK, 128],
    scale uint8 [B, ceil(SK/32), HK, 128]). Runs fmha_mxfp8_quantize_seq32."""
    if x.dim() != 4:
        raise ValueError(f"x: expected [B, SK, HK, 128], got {tuple(x.shape)}")
    B, SK, HK, _ = x.shape
    xb = _bf16(x, "x")
    q = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    sc = torch.empty(B, (SK + 31) // 32, HK, D, dtype=torch.uint8, device=x.device)
    with torch.cuda.device(x.device):
        lib.quantize_seq32(xb.data_ptr(), q.data_ptr(), sc.data_ptr(), B, SK, HK, _cap(xb), _cap(q), _cap(sc), _stream(x.device, stream))
    return q, sc


LOG2E_OVER_SQRT_D = 1.4426950408889634 / math.sqrt(D)


def fmha_fwd_bf16_via_mxfp8(q, k, v, out=None, *, softmax_scale=None, causal=False, path="auto", splits=None, lse=None, stream=None,
                            v_scales="tensor", scale_in_kernel=False):
    """Attention from bf16 q [B, S, H, 128], k / v [B, SK, HK, 128]: quantises on the GPU (Q scaled by
    softmax_scale * log2(e) before quantisation, default 1/sqrt(128), as ref_host.cpp:238 folds it), then runs
    ``fmha_fwd_mxfp8``. Returns out (bf16 [B, S, H, 128]); ``lse``, when given, receives the natural-log LSE of
    the scaled scores. ``v_scales``: "tensor" (one f32 descale, the reference's) or "seq32" (extension: one E8M0 per
    32 keys per column). ``scale_in_kernel`` (extension): Q is quantised as it is and the kernel applies the scale."""
    B, S, H, _ = q.shape
    _, SK, HK, _ = k.shape
    scale = 1.0 / math.sqrt(D) if softmax_scale is None else float(softmax_scale)
    mul = 1.0 if scale_in_kernel else (LOG2E_OVER_SQRT_D if softmax_scale is None else 1.4426950408889634 * scale)
    qs = alloc_scales(B, S, H, q.device)
    ks = alloc_scales(B, SK, HK, k.device)
    q8 = quantize_mxfp8(q, qs, mul=mul, stream=stream)
    k8 = quantize_mxfp8(k, ks, stream=stream)
    if v_scales == "seq32":
        v8, vs = quantize_v_seq32(v, stream=stream)
    elif v_scales == "tensor":
        v8, vs = quantize_v(v, stream=stream)
    else:
        raise ValueError(f"v_scales must be 'tensor' or 'seq32', got {v_scales!r}")
    if out is None:
        out = torch.empty(B, S, H, D, dtype=torch.bfloat16, device=q.device)
    fmha_fwd_mxfp8(q8, k8, v8, qs, ks, vs, out, path=path, splits=splits, stream=stream, lse=lse, causal=causal,
                   softmax_scale=scale if scale_in_kernel else None)
    return out


def random_inputs(B, H, S, SK, HK=None, device="cuda", seed=0):
    """Synthetic MXFP8 inputs with the distribution of the reference's REF_DATA=normal generator
    (N(0,1) Q/K/V, Q x log2(e)/sqrt(128), per-32 E8M0 along head_dim, V e4m3 with one f32 descale), drawn on the
    device with torch's generator in bf16 and quantised by the on-GPU quantisers.
    Returns (q, k, v, q_scale, k_scale, v_scale)."""
    HK = HK or H
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    qs = alloc_scales(B, S, H, device)
    ks = alloc_scales(B, SK, HK, device)
    q = quantize_mxfp8(torch.randn(B, S, H, D, generator=g, device=device, dtype=torch.bfloat16), qs, mul=LOG2E_OVER_SQRT_D)
    k = quantize_mxfp8(torch.randn(B, SK, HK, D, generator=g, device=device, dtype=torch.bfloat16), ks)
    v, vs = quantize_v(torch.randn(B, SK, HK, D, generator=g, device=device, dtype=torch.bfloat16))
    return q, k, v, qs, ks, vs
