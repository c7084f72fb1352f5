"""ctypes binding of the CPU oracle (``oracle/mxfp8_oracle.c``).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py``, always as the checker or the
timed CPU baseline, never as a product path. See ``mxfp8_oracle.h`` for the
reference file:line each function restates.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libmxfp8_oracle.so")
_lib = None

D = 128


def build():
    """Compile the oracle (gcc, no GPU needed)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


class Problem(ctypes.Structure):
    _fields_ = [("B", ctypes.c_int), ("H", ctypes.c_int), ("HK", ctypes.c_int), ("S", ctypes.c_int), ("SK", ctypes.c_int),
                ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
                ("qs", ctypes.c_void_p), ("ks", ctypes.c_void_p), ("vdescale", ctypes.c_float), ("causal", ctypes.c_int),
                ("vs32", ctypes.c_void_p), ("qk_scale", ctypes.c_float)]


class CheckResult(ctypes.Structure):
    _fields_ = [("checked", ctypes.c_uint64), ("bad", ctypes.c_uint64), ("worst_err", ctypes.c_double),
                ("mean_err", ctypes.c_double), ("max_ref", ctypes.c_double)]

    def as_dict(self):
        return {"checked": int(self.checked), "bad": int(self.bad), "worst_err": float(self.worst_err),
                "mean_err": float(self.mean_err), "max_ref": float(self.max_ref)}


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        vp, i, f, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
        L.mxo_e4m3_decode.restype = ctypes.c_double
        L.mxo_e4m3_decode.argtypes = [ctypes.c_uint8]
        L.mxo_e4m3_encode_sat.restype = ctypes.c_uint8
        L.mxo_e4m3_encode_sat.argtypes = [f]
        L.mxo_cvt_bf16_fp8.restype = ctypes.c_uint8
        L.mxo_cvt_bf16_fp8.argtypes = [ctypes.c_uint16, f]
        L.mxo_pknorm_u16.restype = ctypes.c_uint16
        L.mxo_pknorm_u16.argtypes = [f]
        L.mxo_f32_to_f16.restype = ctypes.c_uint16
        L.mxo_f32_to_f16.argtypes = [f]
        L.mxo_f16_to_f32.restype = f
        L.mxo_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.mxo_qs_bytes.restype = sz
        L.mxo_qs_bytes.argtypes = [i, i, i]
        L.mxo_ks_bytes.restype = sz
        L.mxo_ks_bytes.argtypes = [i, i, i, i]
        L.mxo_generate.restype = f
        L.mxo_generate.argtypes = [i, i, i, i, i, i, ctypes.c_uint64, vp, vp, vp, vp, vp]
        L.mxo_select_path.restype = i
        L.mxo_select_path.argtypes = [ctypes.c_long] * 4 + [ctypes.POINTER(i)]
        L.mxo_split_range.restype = None
        L.mxo_split_range.argtypes = [i, i, i, ctypes.POINTER(i), ctypes.POINTER(i)]
        L.mxo_check_fp64.restype = CheckResult
        L.mxo_check_fp64.argtypes = [ctypes.POINTER(Problem), vp, i, i]
        L.mxo_attention_fp32.restype = ctypes.c_double
        L.mxo_attention_fp32.argtypes = [ctypes.POINTER(Problem), i, vp, i]
        L.mxo_emulate.restype = None
        L.mxo_emulate.argtypes = [ctypes.POINTER(Problem), i, i, vp, vp, vp, i]
        L.mxo_combine.restype = None
        L.mxo_combine.argtypes = [vp, vp, vp, ctypes.c_long, i]
        L.mxo_emulate_ex.restype = None
        L.mxo_emulate_ex.argtypes = [ctypes.POINTER(Problem), i, i, vp, vp, vp, i, i, i]
        L.mxo_combine_f32.restype = None
        L.mxo_check_fp64_rows.restype = CheckResult
        L.mxo_check_fp64_rows.argtypes = [ctypes.POINTER(Problem), vp, vp, i, i]
        L.mxo_emulate_rows.restype = None
        L.mxo_emulate_rows.argtypes = [ctypes.POINTER(Problem), i, vp, i, vp, i, i, i]
        L.mxo_combine_f32.argtypes = [vp, vp, vp, ctypes.c_long, i]
        L.mxo_quant_rows_bf16.argtypes = [vp, ctypes.c_long, f, vp, vp]
        L.mxo_quant_rows_bf16.restype = None
        L.mxo_quant_tensor_bf16.argtypes = [vp, ctypes.c_long, vp]
        L.mxo_quant_tensor_bf16.restype = f
        L.mxo_quant_seq32_bf16.argtypes = [vp, i, i, i, vp, vp]
        L.mxo_quant_seq32_bf16.restype = None
        _lib = L
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


MODES = {"lcg": 0, "uniform": 1, "normal": 2}


class Inputs:
    """Seeded MXFP8 inputs in the reference layout (ref_host.cpp:183-263), host numpy arrays."""

    def __init__(self, B, H, S, SK, HK=None, mode="normal", seed_mix=0, causal=False, v_seq32=False, qk_scale=0.0):
        HK = HK or H
        self.B, self.H, self.HK, self.S, self.SK, self.causal = B, H, HK, S, SK, bool(causal)
        # extension: > 0 = the softmax scale applied in the kernel (scores c q.k, c = f32(qk_scale log2 e)); the
        # generator's Q is used as it is
        self.qk_scale = float(qk_scale)
        L = lib()
        self.q = np.zeros(B * S * H * D, np.uint8)
        self.k = np.zeros(B * SK * HK * D, np.uint8)
        self.v = np.zeros(B * SK * HK * D, np.uint8)
        self.qs = np.zeros(L.mxo_qs_bytes(B, H, S), np.uint8)
        self.ks = np.zeros(L.mxo_ks_bytes(B, H, HK, SK), np.uint8)
        self.vdescale = float(L.mxo_generate(MODES[mode], B, H, HK, S, SK, seed_mix, _ptr(self.q), _ptr(self.k),
                                             _ptr(self.v), _ptr(self.qs), _ptr(self.ks)))
        self.vd_buf = np.zeros(1024, np.float32)
        self.vd_buf[0] = self.vdescale
        self.vs32 = None
        if v_seq32:
            # extension: V re-quantised with one E8M0 per 32 keys per column (the seq32 rule) from the generator's V,
            # dequantised and rounded to bf16; the FMHA then reads the scales instead of the f32 descale
            dec = np.array([L.mxo_e4m3_decode(i) for i in range(256)], np.float32)
            vals = dec[self.v] * np.float32(self.vdescale)
            u = vals.view(np.uint32)
            bf = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)    # f32 -> bf16, round to nearest even
            self.v, self.vs32 = quant_seq32_bf16(bf, B, SK, HK)

    def problem(self):
        p = Problem(self.B, self.H, self.HK, self.S, self.SK, _ptr(self.q).value, _ptr(self.k).value, _ptr(self.v).value,
                    _ptr(self.qs).value, _ptr(self.ks).value, self.vdescale, int(self.causal),
                    _ptr(self.vs32).value if self.vs32 is not None else None, self.qk_scale)
        return p

    @property
    def out_elems(self):
        return self.B * self.S * self.H * D


def row_list(S, rows):
    """Normalises a row selection: an int n means the first n rows (as the reference's check samples them); a
    sequence names the rows. Returns an int32 array of distinct rows in [0, S)."""
    if isinstance(rows, (int, np.integer)):
        return np.arange(min(int(rows), S) if rows > 0 else S, dtype=np.int32)
    r = np.unique(np.asarray(rows, dtype=np.int32))
    assert r.size and r.min() >= 0 and r.max() < S, "rows outside [0, S)"
    return r


def first_and_last(S, n=64):
    """The first n and the last n query rows (the reference's 64-row sample plus the end of the sequence: the last
    query tile, the ragged tail and, under the bottom-right causal mask, the rows that see every key tile)."""
    return row_list(S, np.concatenate([np.arange(min(n, S)), np.arange(max(0, S - n), S)]))


def check_fp64(inp, out_bf16, rows=64, threads=0):
    """ref_host.cpp:436-471 statistics of a bf16 output (uint16 array) over `rows` (the first n, or a list)."""
    out = np.ascontiguousarray(out_bf16, dtype=np.uint16).reshape(-1)
    assert out.size == inp.out_elems
    p = inp.problem()
    if isinstance(rows, (int, np.integer)):
        return lib().mxo_check_fp64(ctypes.byref(p), _ptr(out), int(rows), int(threads)).as_dict()
    lst = row_list(inp.S, rows)
    return lib().mxo_check_fp64_rows(ctypes.byref(p), _ptr(out), _ptr(lst), int(lst.size), int(threads)).as_dict()


def emulate(inp, splits=0, rows=64, threads=0, partials=False, f32_partials=False, split_tiles=False):
    """Bit-level model of the reference kernels on the first ``rows`` rows of every (b, h) (or the listed rows).
    Returns the bf16 output (uint16, rows not emulated are 0), and with ``partials`` also (ohat, lse f32): ohat fp16
    (uint16), or f32 with ``f32_partials`` (the FMHA_KVS_F32_PARTIALS extension). ``split_tiles`` models the library's
    order (two 64-key streams per tile, merged; not with the LUT recipe) instead of the reference's: for KV-split blocks
    of at most 128 query rows, and with ``splits=0`` for every row (the t128 path's split-tile kernel). At most 64
    splits."""
    assert 0 <= splits <= 64, f"emulate: {splits} splits (at most 64)"
    out = np.zeros(inp.out_elems, np.uint16)
    if not isinstance(rows, (int, np.integer)):
        assert not partials, "partials are emulated for leading rows only"
        lst = row_list(inp.S, rows)
        lib().mxo_emulate_rows(ctypes.byref(inp.problem()), int(splits), _ptr(lst), int(lst.size), _ptr(out),
                               int(bool(f32_partials)), int(bool(split_tiles)), int(threads))
        return out
    ohat = lse = None
    if partials and splits:
        rows_total = inp.B * inp.S * inp.H
        ohat = np.zeros(splits * rows_total * D, np.float32 if f32_partials else np.uint16)
        lse = np.zeros(splits * rows_total, np.float32)
    p = inp.problem()
    lib().mxo_emulate_ex(ctypes.byref(p), int(splits), int(rows), _ptr(out), _ptr(ohat), _ptr(lse), int(bool(f32_partials)),
                         int(bool(split_tiles)), int(threads))
    return (out, ohat, lse) if partials else out


def attention_fp32(inp, rows=0, threads=0, want_out=True):
    """fp32 attention on the dequantised inputs (the CPU baseline). Returns (seconds, out or None)."""
    out = np.zeros(inp.out_elems, np.float32) if want_out else None
    p = inp.problem()
    secs = lib().mxo_attention_fp32(ctypes.byref(p), int(rows), _ptr(out), int(threads))
    return secs, out


def select_path(B, H, S, SK):
    sp = ctypes.c_int(0)
    path = lib().mxo_select_path(B, H, S, SK, ctypes.byref(sp))
    return ("vs128", "t128", "kvsplit")[path], sp.value


def split_range(SK, splits, s):
    lo, n = ctypes.c_int(0), ctypes.c_int(0)
    lib().mxo_split_range(SK, splits, s, ctypes.byref(lo), ctypes.byref(n))
    return lo.value, n.value


def combine(ohat, lse, rows_total, splits):
    """The combine on partial rows: fp16 (uint16 array) or, for a float32 array, f32 rows (the extension)."""
    out = np.zeros(rows_total * D, np.uint16)
    if np.asarray(ohat).dtype == np.float32:
        lib().mxo_combine_f32(_ptr(np.ascontiguousarray(ohat, np.float32)), _ptr(np.ascontiguousarray(lse, np.float32)),
                              _ptr(out), rows_total, splits)
    else:
        lib().mxo_combine(_ptr(np.ascontiguousarray(ohat, np.uint16)), _ptr(np.ascontiguousarray(lse, np.float32)), _ptr(out),
                          rows_total, splits)
    return out


def bf16_to_f32(a):
    return (np.asarray(a, np.uint16).astype(np.uint32) << 16).view(np.float32)


def quant_rows_bf16(x, mul=1.0):
    """x: uint16 bf16 bits [rows*128] -> (e4m3 bytes [rows*128], E8M0 bytes [rows*4]) by the generator's rule."""
    x = np.ascontiguousarray(x, np.uint16).reshape(-1)
    rows = x.size // D
    q = np.zeros(rows * D, np.uint8)
    sc = np.zeros(rows * 4, np.uint8)
    lib().mxo_quant_rows_bf16(_ptr(x), rows, mul, _ptr(q), _ptr(sc))
    return q, sc


def quant_tensor_bf16(x):
    """x: uint16 bf16 bits [n] -> (e4m3 bytes [n], f32 descale)."""
    x = np.ascontiguousarray(x, np.uint16).reshape(-1)
    q = np.zeros(x.size, np.uint8)
    d = lib().mxo_quant_tensor_bf16(_ptr(x), x.size, _ptr(q))
    return q, np.float32(d)


def quant_seq32_bf16(x, B, SK, HK):
    """x: uint16 bf16 bits [B*SK*HK*128] -> (e4m3 bytes, E8M0 bytes [B*ceil(SK/32)*HK*128])."""
    x = np.ascontiguousarray(x, np.uint16).reshape(-1)
    q = np.zeros(x.size, np.uint8)
    sc = np.zeros(B * ((SK + 31) // 32) * HK * D, np.uint8)
    lib().mxo_quant_seq32_bf16(_ptr(x), B, SK, HK, _ptr(q), _ptr(sc))
    return q, sc
