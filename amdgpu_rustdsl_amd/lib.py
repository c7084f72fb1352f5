"""ctypes binding of the C ABI in include/fmha_mxfp8.h (libfmha_mxfp8.so, built by amdgpu_rustdsl_amd/build.py).

Importing this module loads the native library and raises if it is missing: there is no fallback path.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "libfmha_mxfp8.so")

if not os.path.exists(LIB_PATH):
    raise ImportError(f"{LIB_PATH} is missing: build it with `python amdgpu_rustdsl_amd/build.py` "
                      "(or __graft_entry__.build()); the MXFP8 FMHA has no non-native fallback")

# A process must hold one HIP runtime. PyTorch-ROCm ships its own libamdhip64.so.7 (the same soname as ROCm's), so
# torch, when importable, is imported first: the library then binds to the runtime torch already loaded. Loaded the
# other way round, /opt/rocm's runtime and torch's both come up, and the one that starts second finds no device.
try:
    import torch  # noqa: F401
except ImportError:
    pass

_L = ctypes.CDLL(LIB_PATH)

FMHA_OK, FMHA_ERR_EXTENT, FMHA_ERR_KA_RANGE, FMHA_ERR_KA_IS, FMHA_ERR_GRID, FMHA_ERR_SYM = 0, 1, 2, 3, 4, 5
FMHA_ERR_PATH, FMHA_ERR_WORKSPACE, FMHA_ERR_HIP, FMHA_ERR_NO_DEVICE = 6, 7, 8, 9
PATH_VS128, PATH_T128, PATH_KVSPLIT = 0, 1, 2
KVS_F32_PARTIALS = 0x10000   # include/fmha_mxfp8.h FMHA_KVS_F32_PARTIALS
KVS_V_SEQ32 = 0x20000        # FMHA_KVS_V_SEQ32
KVS_SCALE = 0x40000          # FMHA_KVS_SCALE
FLAG_CAUSAL, FLAG_V_SEQ32, FLAG_SCALE, FLAG_CAUSAL_PAIR = 0x1, 0x2, 0x4, 0x8   # FMHA_FLAG_*
WORKSPACE_SLOTS = 4          # FMHA_WORKSPACE_SLOTS
PATH_NAMES = {PATH_VS128: "vs128", PATH_T128: "t128", PATH_KVSPLIT: "kvsplit"}
PATH_IDS = {v: k for k, v in PATH_NAMES.items()}

_u8, _u32, _u64, _vp = ctypes.c_uint8, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_void_p


def _pad(n):
    return _u8 * n


class Args(ctypes.Structure):
    """fmha_mxfp8_args: the 656-byte kernarg of _vs128 / _t128 (field names of the reference's generated Args)."""
    _pack_ = 1
    _fields_ = [("ptr_o", _vp), ("_pad0", _pad(8)), ("ptr_q", _vp), ("_pad1", _pad(8)), ("ptr_k", _vp), ("_pad2", _pad(8)),
                ("ptr_v", _vp), ("_pad3", _pad(8)), ("ptr_lse", _vp), ("_pad3b", _pad(8)), ("softmax_scale", _u32),
                ("_pad3c", _pad(12)), ("s_seq_len", _u32), ("_pad4", _pad(12)), ("s_Seqs", _u32), ("_pad5", _pad(28)),
                ("s_Hs", _u32), ("_pad6", _pad(12)), ("s_Bs", _u32), ("_pad7", _pad(12)), ("s_gqa", _u32), ("_pad8", _pad(12)),
                ("s_k_Seqs", _u32), ("_pad9", _pad(12)), ("s_k_Hs", _u32), ("_pad10", _pad(12)), ("s_k_Bs", _u32),
                ("_pad11", _pad(12)), ("opt", _u32), ("_pad11b", _pad(28)), ("s_kv_seq_len", _u32), ("_pad12", _pad(44)),
                ("s_q_head_num", _u32), ("_pad13", _pad(12)), ("s_v_Seqs", _u32), ("_pad14", _pad(12)), ("s_v_Hs", _u32),
                ("_pad15", _pad(12)), ("s_v_Bs", _u32), ("_pad16", _pad(12)), ("s_o_Seqs", _u32), ("_pad17", _pad(12)),
                ("s_o_Hs", _u32), ("_pad18", _pad(12)), ("s_o_Bs", _u32), ("_pad19", _pad(92)), ("ptr_q_descale", _vp),
                ("_pad20", _pad(8)), ("ptr_k_descale", _vp), ("_pad21", _pad(8)), ("ptr_v_descale", _vp), ("_pad22", _pad(8)),
                ("s_descale_q_Bs", _u32), ("_pad23", _pad(12)), ("s_descale_q_Hs", _u32), ("_pad24", _pad(12)),
                ("s_descale_k_Bs", _u32), ("_pad25", _pad(12)), ("s_descale_k_Hs", _u32), ("_pad26", _pad(28)),
                ("flags", _u32), ("abi_tail", _pad(12))]


class KvsplitArgs(ctypes.Structure):
    """fmha_mxfp8_kvsplit_args: 648 bytes (base layout to 0x270, then the split extension)."""
    _pack_ = 1
    _fields_ = [("base", _pad(0x270)), ("ptr_ohat", _vp), ("ptr_lse", _vp), ("kvs_splits", _u32), ("kvs_rows_total", _u32)]


class CombineArgs(ctypes.Structure):
    _pack_ = 1
    _fields_ = [("ptr_ohat", _vp), ("ptr_lse", _vp), ("ptr_out", _vp), ("rows_total", _u32), ("d", _u32), ("splits", _u32)]


class BufferSizes(ctypes.Structure):
    _fields_ = [(n, _u64) for n in ("ptr_q", "ptr_k", "ptr_v", "ptr_o", "ptr_q_descale", "ptr_k_descale", "ptr_v_descale",
                                    "ptr_ohat", "ptr_lse")]


class Params(ctypes.Structure):
    _fields_ = [("o", _vp), ("q", _vp), ("k", _vp), ("v", _vp), ("q_descale", _vp), ("k_descale", _vp), ("v_descale", _vp),
                ("lse", _vp), ("bytes_q", _u64), ("bytes_k", _u64), ("bytes_v", _u64), ("bytes_o", _u64),
                ("bytes_q_descale", _u64), ("bytes_k_descale", _u64), ("bytes_v_descale", _u64),
                ("B", ctypes.c_int32), ("H", ctypes.c_int32), ("HK", ctypes.c_int32), ("S", ctypes.c_int32), ("SK", ctypes.c_int32),
                ("path", ctypes.c_int32), ("splits", ctypes.c_int32), ("causal", ctypes.c_int32),
                ("f32_partials", ctypes.c_int32), ("v_seq32", ctypes.c_int32), ("softmax_scale", ctypes.c_float),
                ("no_check", ctypes.c_int32), ("causal_pair", ctypes.c_int32), ("kv_fill", ctypes.c_int32),
                ("ws_turn", ctypes.POINTER(ctypes.c_uint32)), ("partials_out", ctypes.POINTER(ctypes.c_int32))]


assert ctypes.sizeof(Params) == 192 and ctypes.sizeof(Args) == 656 and ctypes.sizeof(KvsplitArgs) == 648 and ctypes.sizeof(CombineArgs) == 36

_c, _i64, _sz, _cp = ctypes.c_int, ctypes.c_int64, ctypes.c_size_t, ctypes.c_char_p
_P = ctypes.POINTER
_L.fmha_mxfp8_validate_vs128.argtypes = [_P(Args), _P(BufferSizes), _u32, _u32, _u32, _i64, _cp, _sz]
_L.fmha_mxfp8_validate_t128.argtypes = [_P(Args), _P(BufferSizes), _u32, _u32, _u32, _i64, _cp, _sz]
_L.fmha_mxfp8_validate_kvsplit.argtypes = [_P(KvsplitArgs), _P(BufferSizes), _u32, _u32, _u32, _i64, _i64, _i64, _cp, _sz]
_L.fmha_mxfp8_validate_combine.argtypes = [_P(CombineArgs), _P(BufferSizes), _u32, _u32, _u32, _cp, _sz]
_L.fmha_mxfp8_select_path.argtypes = [_i64, _i64, _i64, _i64, _P(_c)]
_L.fmha_mxfp8_uses_split_tiles.argtypes = [_c, _i64, _i64, _i64, _i64, _c]
_L.fmha_mxfp8_fill_args.argtypes = [_P(Args), _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c, _c, _c, _c, _c]
_L.fmha_mxfp8_fill_args.restype = None
_L.fmha_mxfp8_workspace_bytes.argtypes = [_i64, _i64, _i64, _c]
_L.fmha_mxfp8_workspace_bytes.restype = _sz
_L.fmha_mxfp8_kv_partials.argtypes = [_i64, _i64, _i64, _i64, _c]
_L.fmha_mxfp8_launch_vs128.argtypes = [_P(Args), _u32, _u32, _u32, _vp]
_L.fmha_mxfp8_launch_t128.argtypes = [_P(Args), _u32, _u32, _u32, _vp]
_L.fmha_mxfp8_launch_t128_split_tiles.argtypes = [_P(Args), _u32, _u32, _u32, _vp]
_L.fmha_mxfp8_launch_kvsplit.argtypes = [_P(KvsplitArgs), _u32, _u32, _u32, _vp]
_L.fmha_mxfp8_launch_combine.argtypes = [_P(CombineArgs), _u32, _vp]
_L.fmha_mxfp8_launch_combine_wide.argtypes = [_P(CombineArgs), _u32, _vp]
_L.fmha_fwd_hd128_mxfp8_auto.argtypes = [_P(Params), _vp, _sz, _vp, _P(_c), _P(_c), _cp, _sz]
_L.fmha_fwd_hd128_mxfp8_auto_noalloc.argtypes = [_P(Params), _vp, _P(_c), _P(_c), _cp, _sz]
_L.fmha_mxfp8_init.argtypes = [_cp, _sz]
_L.fmha_mxfp8_version.restype = _cp
_L.fmha_mxfp8_version.argtypes = []
# include/mxfp8_quant.h
_L.fmha_mxfp8_quantize_rows.argtypes = [_vp, _vp, _vp, _i64, ctypes.c_float, _u64, _u64, _u64, _vp, _cp, _sz]
_L.fmha_mxfp8_quantize_tensor.argtypes = [_vp, _vp, _vp, _i64, _u64, _u64, _u64, _vp, _cp, _sz]
_L.fmha_mxfp8_quantize_seq32.argtypes = [_vp, _vp, _vp, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, _u64, _u64, _u64, _vp, _cp, _sz]
_L.fmha_mxfp8_seq32_scale_bytes.argtypes = [_i64, _i64, _i64]
_L.fmha_mxfp8_seq32_scale_bytes.restype = _sz

EXPORTED = ["fmha_mxfp8_validate_vs128", "fmha_mxfp8_validate_t128", "fmha_mxfp8_validate_kvsplit", "fmha_mxfp8_validate_combine",
            "fmha_mxfp8_select_path", "fmha_mxfp8_uses_split_tiles", "fmha_mxfp8_fill_args", "fmha_mxfp8_workspace_bytes", "fmha_mxfp8_kv_partials", "fmha_mxfp8_launch_vs128",
            "fmha_mxfp8_launch_t128", "fmha_mxfp8_launch_t128_split_tiles", "fmha_mxfp8_launch_kvsplit", "fmha_mxfp8_launch_combine", "fmha_mxfp8_launch_combine_wide", "fmha_fwd_hd128_mxfp8_auto",
            "fmha_fwd_hd128_mxfp8_auto_noalloc",
            "fmha_mxfp8_init", "fmha_mxfp8_version",
            "fmha_mxfp8_quantize_rows", "fmha_mxfp8_quantize_tensor", "fmha_mxfp8_quantize_seq32", "fmha_mxfp8_seq32_scale_bytes"]

raw = _L


class FmhaError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(msg)
        self.code = code


def _errbuf():
    return ctypes.create_string_buffer(512)


def check(rc, buf):
    if rc != FMHA_OK:
        raise FmhaError(rc, buf.value.decode(errors="replace") or f"fmha error {rc}")


def select_path(B, H, S, SK):
    sp = ctypes.c_int(0)
    path = _L.fmha_mxfp8_select_path(B, H, S, SK, ctypes.byref(sp))
    return PATH_NAMES[path], sp.value


def uses_split_tiles(path, B, H, S, SK, causal=False):
    """Whether the one-call entry runs the full-sequence `path` ("vs128" / "t128") on the split-tile kernel."""
    if path not in ("vs128", "t128"):
        return False
    return bool(_L.fmha_mxfp8_uses_split_tiles(PATH_IDS[path], B, H, S, SK, int(bool(causal))))


def workspace_bytes(B, H, S, splits):
    return int(_L.fmha_mxfp8_workspace_bytes(B, H, S, splits))


def kv_partials(B, H, S, SK, splits):
    """Partials per row the one-call entry writes for a KV split of ``splits`` chunks when the workspace holds them
    (the chunks times the fill that spreads each chunk over up to 8 blocks; the current device's CU count)."""
    return int(_L.fmha_mxfp8_kv_partials(B, H, S, SK, splits))


def fill_args(o, q, k, v, qs, ks, vs, B, H, HK, S, SK):
    a = Args()
    _L.fmha_mxfp8_fill_args(ctypes.byref(a), o, q, k, v, qs, ks, vs, B, H, HK, S, SK)
    return a


def validate(kind, args, sizes, grid, **syms):
    """validate(): returns (code, message). kind: vs128 | t128 | kvsplit | combine."""
    buf = _errbuf()
    gx, gy, gz = grid
    if kind == "vs128":
        rc = _L.fmha_mxfp8_validate_vs128(ctypes.byref(args), ctypes.byref(sizes), gx, gy, gz, syms.get("HK", 1), buf, 512)
    elif kind == "t128":
        rc = _L.fmha_mxfp8_validate_t128(ctypes.byref(args), ctypes.byref(sizes), gx, gy, gz, syms.get("HK", 1), buf, 512)
    elif kind == "kvsplit":
        rc = _L.fmha_mxfp8_validate_kvsplit(ctypes.byref(args), ctypes.byref(sizes), gx, gy, gz, syms.get("B", 1), syms.get("HK", 1),
                                            syms.get("KL", 0), buf, 512)
    elif kind == "combine":
        rc = _L.fmha_mxfp8_validate_combine(ctypes.byref(args), ctypes.byref(sizes), gx, gy, gz, buf, 512)
    else:
        raise ValueError(kind)
    return rc, buf.value.decode()


def init():
    buf = _errbuf()
    check(_L.fmha_mxfp8_init(buf, 512), buf)


class Ran(tuple):
    """(path name, splits) of a one-call entry: the KV split's chunk count, as the reference op returns it. The
    partials per row that ran (the chunks times the KV fill) are in ``.partials`` (0 off the KV split)."""

    def __new__(cls, path, splits, partials):
        r = super().__new__(cls, (path, splits))
        r.partials = partials
        return r


def _run(entry, params, *args):
    buf = _errbuf()
    path, splits = ctypes.c_int(-1), ctypes.c_int(0)
    own = not params.partials_out
    parts = ctypes.c_int32(0)
    if own:
        params.partials_out = ctypes.pointer(parts)
    try:
        rc = entry(ctypes.byref(params), *args, ctypes.byref(path), ctypes.byref(splits), buf, 512)
        n = params.partials_out[0]
    finally:
        if own:
            params.partials_out = None
    check(rc, buf)
    return Ran(PATH_NAMES[path.value], splits.value, n)


def run_auto(params, workspace=None, workspace_bytes=0, stream=None):
    """fmha_fwd_hd128_mxfp8_auto; returns Ran (path name, splits; .partials)."""
    return _run(_L.fmha_fwd_hd128_mxfp8_auto, params, workspace, workspace_bytes, stream)


NOALLOC_SCRATCH_BYTES = 33816576   # FMHA_NOALLOC_SCRATCH_BYTES


def run_auto_noalloc(params, stream=None):
    """fmha_fwd_hd128_mxfp8_auto_noalloc (no workspace argument); returns Ran (path name, splits; .partials)."""
    return _run(_L.fmha_fwd_hd128_mxfp8_auto_noalloc, params, stream)


def quantize_rows(x, q, scale, rows, mul, bytes_x, bytes_q, bytes_scale, stream=None):
    buf = _errbuf()
    check(_L.fmha_mxfp8_quantize_rows(x, q, scale, rows, mul, bytes_x, bytes_q, bytes_scale, stream, buf, 512), buf)


def quantize_tensor(x, q, descale, n, bytes_x, bytes_q, bytes_descale, stream=None):
    buf = _errbuf()
    check(_L.fmha_mxfp8_quantize_tensor(x, q, descale, n, bytes_x, bytes_q, bytes_descale, stream, buf, 512), buf)


def quantize_seq32(x, q, scale, B, SK, HK, bytes_x, bytes_q, bytes_scale, stream=None):
    buf = _errbuf()
    check(_L.fmha_mxfp8_quantize_seq32(x, q, scale, B, SK, HK, bytes_x, bytes_q, bytes_scale, stream, buf, 512), buf)


def seq32_scale_bytes(B, SK, HK):
    return int(_L.fmha_mxfp8_seq32_scale_bytes(B, SK, HK))
