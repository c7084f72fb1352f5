"""CPU tests of the drop-in boundary (include/fmha_mxfp8.h, libfmha_mxfp8.so): the library loads without a GPU, exports
every declared entry point, lays the kernargs out at the reference's offsets, and its host contract (validate, path
selection, workspace size, argument errors of the auto entry) behaves as the reference's
(tests/gpu/generated/fmha_fwd_hd128_mxfp8_v3_vs128_abi.h:10-209, kvsplit / combine8h headers,
crates/amdgpu-graph/src/dispatch.rs:494-511). No test here launches a kernel."""
import ctypes
import math
import struct
import os
import re

import pytest

import oracle
from amdgpu_rustdsl_amd import lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in ("fmha_mxfp8.h", "mxfp8_quant.h")]


def _declared_functions():
    src = "\n".join(open(h).read() for h in HEADERS)
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    src = re.sub(r"//[^\n]*", "", src)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(fmha_\w+)\s*\(", src, flags=re.M)))


def test_every_declared_symbol_is_exported():
    names = _declared_functions()
    assert "fmha_fwd_hd128_mxfp8_auto" in names and len(names) >= 14
    for n in names:
        assert hasattr(lib.raw, n), f"{n} declared in include/ but not exported"
    assert sorted(lib.EXPORTED) == names


def test_header_constants_match_the_binding():
    """The flag bits and sizes the ctypes binding uses are the header's #defines."""
    src = open(HEADERS[0]).read()
    defs = {m.group(1): int(m.group(2), 0) for m in re.finditer(r"#define (FMHA_\w+) (0x[0-9a-fA-F]+|\d+)u?", src)}
    assert defs["FMHA_FLAG_CAUSAL"] == lib.FLAG_CAUSAL and defs["FMHA_FLAG_V_SEQ32"] == lib.FLAG_V_SEQ32
    assert defs["FMHA_FLAG_SCALE"] == lib.FLAG_SCALE and defs["FMHA_FLAG_CAUSAL_PAIR"] == lib.FLAG_CAUSAL_PAIR
    assert defs["FMHA_KVS_V_SEQ32"] == lib.KVS_V_SEQ32 and defs["FMHA_KVS_SCALE"] == lib.KVS_SCALE
    assert defs["FMHA_WORKSPACE_SLOTS"] == lib.WORKSPACE_SLOTS
    assert defs["FMHA_NOALLOC_SCRATCH_BYTES"] == lib.NOALLOC_SCRATCH_BYTES


def test_version_string():
    assert lib.raw.fmha_mxfp8_version().decode().startswith("fmha_mxfp8 gfx950")


# vs128_abi.h:10-126 (Args), kvsplit_abi.h (0x270-0x287), combine8h_abi.h (36 B)
OFFSETS = {
    "ptr_o": 0x000, "ptr_q": 0x010, "ptr_k": 0x020, "ptr_v": 0x030, "ptr_lse": 0x040, "softmax_scale": 0x050,
    "s_seq_len": 0x060, "s_Seqs": 0x070, "s_Hs": 0x090, "s_Bs": 0x0A0, "s_gqa": 0x0B0, "s_k_Seqs": 0x0C0,
    "s_k_Hs": 0x0D0, "s_k_Bs": 0x0E0, "opt": 0x0F0, "s_kv_seq_len": 0x110, "s_q_head_num": 0x140, "s_v_Seqs": 0x150,
    "s_v_Hs": 0x160, "s_v_Bs": 0x170, "s_o_Seqs": 0x180, "s_o_Hs": 0x190, "s_o_Bs": 0x1A0, "ptr_q_descale": 0x200,
    "ptr_k_descale": 0x210, "ptr_v_descale": 0x220, "s_descale_q_Bs": 0x230, "s_descale_q_Hs": 0x240,
    "s_descale_k_Bs": 0x250, "s_descale_k_Hs": 0x260, "flags": 0x280,
}


def test_kernarg_layouts():
    assert ctypes.sizeof(lib.Args) == 656 and ctypes.sizeof(lib.KvsplitArgs) == 648 and ctypes.sizeof(lib.CombineArgs) == 36
    for name, off in OFFSETS.items():
        assert getattr(lib.Args, name).offset == off, name
    assert lib.KvsplitArgs.ptr_ohat.offset == 0x270 and lib.KvsplitArgs.ptr_lse.offset == 0x278
    assert lib.KvsplitArgs.kvs_splits.offset == 0x280 and lib.KvsplitArgs.kvs_rows_total.offset == 0x284
    assert [lib.CombineArgs.ptr_ohat.offset, lib.CombineArgs.ptr_lse.offset, lib.CombineArgs.ptr_out.offset,
            lib.CombineArgs.rows_total.offset, lib.CombineArgs.d.offset, lib.CombineArgs.splits.offset] == [0, 8, 16, 24, 28, 32]


def _shape_args(B=2, H=8, HK=4, S=300, SK=700):
    a = lib.fill_args(0x1000, 0x2000, 0x3000, 0x4000, 0x5000, 0x6000, 0x7000, B, H, HK, S, SK)
    sz = lib.BufferSizes(B * S * H * 128, B * SK * HK * 128, B * SK * HK * 128, B * S * H * 256,
                         B * S * H * 4 + 2048 * H, B * SK * HK * 4 + 2560 * H, 4096, 0, 0)
    return a, sz


def test_fill_args_values():
    """ref_host.cpp:272-330 packing: strides in bytes, head strides 128 / 256 / 4, gqa = H / HK, opt = 5."""
    B, H, HK, S, SK = 2, 8, 4, 300, 700
    a, _ = _shape_args(B, H, HK, S, SK)
    assert (a.ptr_o, a.ptr_q, a.ptr_k, a.ptr_v, a.ptr_q_descale, a.ptr_k_descale, a.ptr_v_descale) == \
        (0x1000, 0x2000, 0x3000, 0x4000, 0x5000, 0x6000, 0x7000)
    assert (a.s_seq_len, a.s_kv_seq_len, a.s_q_head_num, a.s_gqa) == (S, SK, H, H // HK)
    assert (a.s_Seqs, a.s_Hs, a.s_Bs) == (H * 128, 128, S * H * 128)
    assert (a.s_k_Seqs, a.s_k_Hs, a.s_k_Bs) == (HK * 128, 128, SK * HK * 128)
    assert (a.s_v_Seqs, a.s_v_Hs, a.s_v_Bs) == (HK * 128, 128, SK * HK * 128)
    assert (a.s_o_Seqs, a.s_o_Hs, a.s_o_Bs) == (H * 256, 256, S * H * 256)
    assert (a.s_descale_q_Bs, a.s_descale_q_Hs, a.s_descale_k_Bs, a.s_descale_k_Hs) == (S * H * 4, 4, SK * HK * 4, 4)
    assert a.flags == 0 and a.ptr_lse is None


@pytest.mark.parametrize("kind,rows", [("vs128", 256), ("t128", 128)])
def test_validate_accepts_consistent_launch(kind, rows):
    a, sz = _shape_args()
    assert lib.validate(kind, a, sz, (math.ceil(300 / rows), 8, 2), HK=4) == (0, "")


# (mutation, expected code, message fragment) in the reference's rule order
NEGATIVE = [
    (lambda a, sz, g: setattr(sz, "ptr_q", sz.ptr_q - 1), lib.FMHA_ERR_EXTENT, "ptr_q"),
    (lambda a, sz, g: setattr(sz, "ptr_o", 10), lib.FMHA_ERR_EXTENT, "ptr_o"),
    (lambda a, sz, g: setattr(sz, "ptr_q_descale", sz.ptr_q_descale - 1), lib.FMHA_ERR_EXTENT, "ptr_q_descale"),
    (lambda a, sz, g: setattr(sz, "ptr_k_descale", sz.ptr_k_descale - 1), lib.FMHA_ERR_EXTENT, "ptr_k_descale"),
    (lambda a, sz, g: setattr(sz, "ptr_v_descale", 4095), lib.FMHA_ERR_EXTENT, "ptr_v_descale"),
    (lambda a, sz, g: setattr(a, "s_gqa", 0), lib.FMHA_ERR_KA_RANGE, "0xB0"),
    (lambda a, sz, g: setattr(a, "s_gqa", 32), lib.FMHA_ERR_KA_RANGE, "0xB0"),
    (lambda a, sz, g: setattr(a, "s_Hs", 64), lib.FMHA_ERR_KA_RANGE, "0x90"),
    (lambda a, sz, g: setattr(a, "s_o_Hs", 128), lib.FMHA_ERR_KA_RANGE, "0x190"),
    (lambda a, sz, g: setattr(a, "s_descale_k_Hs", 8), lib.FMHA_ERR_KA_RANGE, "0x260"),
    (lambda a, sz, g: setattr(a, "s_gqa", 4), lib.FMHA_ERR_KA_IS, "0x140"),
    (lambda a, sz, g: setattr(a, "s_Seqs", 1000), lib.FMHA_ERR_KA_IS, "0x70"),
    (lambda a, sz, g: setattr(a, "s_v_Seqs", 128), lib.FMHA_ERR_KA_IS, "0x150"),
    (lambda a, sz, g: setattr(a, "s_descale_k_Bs", 4), lib.FMHA_ERR_KA_IS, "0x250"),
    (lambda a, sz, g: g.__setitem__(1, 7), lib.FMHA_ERR_GRID, "axis 1"),
    (lambda a, sz, g: g.__setitem__(0, 1), lib.FMHA_ERR_GRID, "axis 0"),
]


@pytest.mark.parametrize("i", range(len(NEGATIVE)))
def test_validate_rejects(i):
    mutate, code, frag = NEGATIVE[i]
    a, sz = _shape_args()
    g = [math.ceil(300 / 256), 8, 2]
    mutate(a, sz, g)
    rc, msg = lib.validate("vs128", a, sz, tuple(g), HK=4)
    assert rc == code and frag in msg, (rc, msg)
    assert msg.startswith("GV-HOST-")


def _kvsplit(B=1, H=8, HK=8, S=128, SK=16384, splits=8):
    a, sz = _shape_args(B, H, HK, S, SK)
    ka = lib.KvsplitArgs()
    ctypes.memmove(ctypes.addressof(ka), ctypes.addressof(a), 0x270)
    rows = B * S * H
    ka.ptr_ohat, ka.ptr_lse, ka.kvs_splits, ka.kvs_rows_total = 0x8000, 0x9000, splits, rows
    sz.ptr_ohat, sz.ptr_lse = splits * rows * 512, splits * rows * 4
    return ka, sz, (math.ceil(S / 256), H, B * splits)


def test_validate_kvsplit():
    ka, sz, g = _kvsplit()
    assert lib.validate("kvsplit", ka, sz, g, B=1, HK=8, KL=0) == (0, "")
    ka2, sz2, _ = _kvsplit()
    sz2.ptr_ohat -= 1
    assert lib.validate("kvsplit", ka2, sz2, g, B=1, HK=8)[0] == lib.FMHA_ERR_EXTENT
    ka3, sz3, _ = _kvsplit()
    ka3.kvs_rows_total += 1
    rc, msg = lib.validate("kvsplit", ka3, sz3, g, B=1, HK=8)
    assert rc == lib.FMHA_ERR_EXTENT or (rc == lib.FMHA_ERR_KA_IS and "0x284" in msg)
    ka4, sz4, _ = _kvsplit()
    ka4.kvs_rows_total += 1
    sz4.ptr_ohat, sz4.ptr_lse = 1 << 40, 1 << 40
    rc, msg = lib.validate("kvsplit", ka4, sz4, g, B=1, HK=8)
    assert rc == lib.FMHA_ERR_KA_IS and "0x284" in msg
    ka5, sz5, _ = _kvsplit()
    assert lib.validate("kvsplit", ka5, sz5, (g[0], g[1], 4), B=1, HK=8)[0] == lib.FMHA_ERR_GRID
    ka6, sz6, _ = _kvsplit()
    ka6.kvs_splits = 0
    assert lib.validate("kvsplit", ka6, sz6, g, B=1, HK=8)[0] == lib.FMHA_ERR_KA_RANGE
    assert lib.validate("kvsplit", ka, sz, g, B=1, HK=8, KL=-1)[0] == lib.FMHA_ERR_SYM


def test_validate_f32_partials_flag():
    """The f32-partials extension rides in bit 16 of the split fields (kvsplit 0x280, combine 0x20): accepted with the
    split count in the low 16 bits, which the grid relation uses; any other high bit is out of contract."""
    ka, sz, g = _kvsplit()
    ka.kvs_splits = 8 | lib.KVS_F32_PARTIALS
    assert lib.validate("kvsplit", ka, sz, g, B=1, HK=8, KL=0) == (0, "")
    ka.kvs_splits = 8 | (1 << 19)
    rc, msg = lib.validate("kvsplit", ka, sz, g, B=1, HK=8)
    assert rc == lib.FMHA_ERR_KA_RANGE and "0x280" in msg
    ca = lib.CombineArgs(0x1, 0x2, 0x3, 1024, 128, 8 | lib.KVS_F32_PARTIALS)
    csz = lib.BufferSizes(0, 0, 0, 1024 * 256, 0, 0, 0, 8 * 1024 * 512, 8 * 1024 * 4)
    assert lib.validate("combine", ca, csz, (64, 1, 1)) == (0, "")
    ca.splits = 8 | (1 << 20)
    assert lib.validate("combine", ca, csz, (64, 1, 1))[0] == lib.FMHA_ERR_KA_RANGE


def test_validate_v_seq32_flag():
    """Per-32-key V scales (extension, flags bit 1 / kvs_splits bit 17): ptr_v_descale must then hold the E8M0 tensor
    [B, ceil(SK/32), HK, 128] instead of 4 KiB; unknown flag bits are out of contract."""
    B, H, HK, S, SK = 2, 8, 4, 300, 1000
    a, sz = _shape_args(B, H, HK, S, SK)
    grid = (math.ceil(S / 256), H, B)
    need = B * math.ceil(SK / 32) * HK * 128
    a.flags = lib.FLAG_V_SEQ32
    sz.ptr_v_descale = need
    assert lib.validate("vs128", a, sz, grid, HK=HK) == (0, "")
    sz.ptr_v_descale = need - 1
    assert lib.validate("vs128", a, sz, grid, HK=HK)[0] == lib.FMHA_ERR_EXTENT
    sz.ptr_v_descale = need
    a.flags = lib.FLAG_V_SEQ32 | lib.FLAG_CAUSAL
    assert lib.validate("vs128", a, sz, grid, HK=HK) == (0, "")
    a.flags = 0x8
    rc, msg = lib.validate("vs128", a, sz, grid, HK=HK)
    assert rc == lib.FMHA_ERR_KA_RANGE and "0x280" in msg
    ka, ksz, g = _kvsplit(B=1, H=8, HK=8, S=128, SK=16384, splits=8)
    ka.kvs_splits = 8 | lib.KVS_V_SEQ32
    ksz.ptr_v_descale = 4096
    assert lib.validate("kvsplit", ka, ksz, g, B=1, HK=8)[0] == lib.FMHA_ERR_EXTENT
    ksz.ptr_v_descale = 16384 // 32 * 8 * 128
    assert lib.validate("kvsplit", ka, ksz, g, B=1, HK=8, KL=0) == (0, "")


def test_validate_combine():
    ca = lib.CombineArgs(0x1, 0x2, 0x3, 1024, 128, 8)
    sz = lib.BufferSizes(0, 0, 0, 1024 * 256, 0, 0, 0, 8 * 1024 * 512, 8 * 1024 * 4)
    assert lib.validate("combine", ca, sz, (64, 1, 1)) == (0, "")
    ca.d = 64
    assert lib.validate("combine", ca, sz, (64, 1, 1))[0] == lib.FMHA_ERR_KA_RANGE
    ca.d = 128
    sz.ptr_o -= 1
    assert lib.validate("combine", ca, sz, (64, 1, 1))[0] == lib.FMHA_ERR_EXTENT


def test_select_path_matches_oracle():
    """The host dispatch (C++) and the oracle's restatement (C) agree on a grid of shapes, including the empty-split
    exclusion (dispatch.rs:494-511)."""
    for B in (1, 2, 3, 4, 8):
        for H in (1, 2, 8, 16, 64):
            for S in (1, 77, 128, 256, 257, 1000, 2048, 8192):
                for SK in (1, 100, 1337, 2048, 2049, 4096, 16000, 16384, 20000):
                    assert lib.select_path(B, H, S, SK) == oracle.select_path(B, H, S, SK), (B, H, S, SK)
    # published choices (docs/perf-matrix.md:31-55)
    assert lib.select_path(1, 8, 2048, 2048) == ("kvsplit", 4)
    assert lib.select_path(1, 8, 4096, 4096) == ("kvsplit", 2)
    assert lib.select_path(4, 8, 2048, 2048)[0] == "vs128"
    assert lib.select_path(4, 8, 512, 512)[0] == "t128"
    assert lib.select_path(1, 8, 128, 16384) == ("kvsplit", 4)


def test_uses_split_tiles_rule():
    """Which full-sequence launches of the one-call entry run on the split-tile kernel: t128 from 7 key tiles on (4
    with the causal mask); vs128 from the same counts when its 256-row grid holds at most 128 blocks (always with
    the causal mask); never the KV split's own kernel. Below the threshold the 256-thread t128 kernel runs."""
    assert not lib.uses_split_tiles("t128", 1, 8, 512, 512)        # 4 key tiles: the single-wave kernel is faster
    assert not lib.uses_split_tiles("t128", 1, 8, 512, 768)        # 6
    assert lib.uses_split_tiles("t128", 1, 8, 512, 769)            # 7
    assert lib.uses_split_tiles("t128", 1, 8, 512, 512, causal=True)
    assert not lib.uses_split_tiles("t128", 1, 8, 100, 384, causal=True)   # 3 key tiles: LUT recipe
    assert not lib.uses_split_tiles("t128", 1, 1, 256, 256)        # 2 key tiles: LUT recipe
    # causal grids that the pairing halves (more 128-row blocks than CUs) with at most 8 key tiles: single-wave
    assert not lib.uses_split_tiles("t128", 16, 8, 512, 512, causal=True)
    assert not lib.uses_split_tiles("vs128", 8, 8, 1024, 1024, causal=True)
    assert lib.uses_split_tiles("vs128", 8, 8, 1152, 1152, causal=True)      # 9 key tiles
    assert lib.uses_split_tiles("vs128", 4, 8, 1024, 1024, causal=True)      # 256 blocks: not paired
    assert not lib.uses_split_tiles("vs128", 4, 8, 2048, 2048)     # 256 blocks: the whole chip already
    assert lib.uses_split_tiles("vs128", 2, 8, 2048, 2048)         # 128 blocks
    assert lib.uses_split_tiles("vs128", 4, 8, 1024, 1024)
    assert not lib.uses_split_tiles("vs128", 8, 8, 512, 512)       # 4 key tiles: on the 256-thread kernel
    assert lib.uses_split_tiles("vs128", 8, 8, 512, 1024)
    assert not lib.uses_split_tiles("vs128", 2, 8, 2100, 1000)     # 9 x 8 x 2 = 144 blocks
    assert not lib.uses_split_tiles("vs128", 1, 8, 8192, 8192)
    assert not lib.uses_split_tiles("kvsplit", 1, 8, 2048, 2048)
    for B, H, S, SK in ((1, 8, 2048, 2048), (2, 8, 2048, 2048), (4, 8, 512, 512), (3, 5, 777, 1500), (1, 1, 1, 1),
                        (1, 8, 1024, 896)):
        path = lib.select_path(B, H, S, SK)[0]
        blocks256 = (S + 255) // 256 * H * B
        ntiles = (SK + 127) // 128
        want = path in ("t128", "vs128") and ntiles >= 7 and (path == "t128" or blocks256 <= 128)
        assert lib.uses_split_tiles(path, B, H, S, SK) == want, (B, H, S, SK)


def test_workspace_bytes():
    for B, H, S, sp in ((1, 8, 128, 8), (4, 8, 2048, 2), (3, 5, 77, 4)):
        assert lib.workspace_bytes(B, H, S, sp) == sp * B * S * H * (512 + 4)


def _params(**kw):
    p = lib.Params()
    p.B, p.H, p.HK, p.S, p.SK = kw.get("B", 1), kw.get("H", 8), kw.get("HK", 8), kw.get("S", 128), kw.get("SK", 4096)
    p.path, p.splits, p.causal = kw.get("path", -1), kw.get("splits", 0), kw.get("causal", 0)
    p.kv_fill = kw.get("kv_fill", 0)
    big = 1 << 40
    p.o = p.q = p.k = p.v = p.q_descale = p.k_descale = p.v_descale = 0x1000
    p.bytes_q = p.bytes_k = p.bytes_v = p.bytes_o = p.bytes_q_descale = p.bytes_k_descale = p.bytes_v_descale = big
    return p


@pytest.mark.parametrize("kw,code", [
    (dict(H=6, HK=4), lib.FMHA_ERR_KA_RANGE),              # H not a power-of-two multiple of HK
    (dict(H=64, HK=2), lib.FMHA_ERR_KA_RANGE),             # gqa 32 > 16
    (dict(S=0), lib.FMHA_ERR_KA_RANGE),
    (dict(path=7), lib.FMHA_ERR_PATH),
    (dict(path=2, splits=3), lib.FMHA_ERR_PATH),            # splits not in {2, 4, 8}
    (dict(path=2, splits=8, SK=4224), lib.FMHA_ERR_PATH),   # 33 tiles, 5 per split: split 7 would start past the end
    (dict(path=2, splits=4, causal=1), lib.FMHA_ERR_PATH),  # no causal on the KV split
    (dict(kv_fill=2), lib.FMHA_ERR_KA_RANGE),               # kv_fill is 0 or 1
])
def test_auto_rejects_before_any_gpu_work(kw, code):
    """fmha_fwd_hd128_mxfp8_auto checks its arguments before touching the device (these run without a GPU)."""
    p = _params(**kw)
    err = ctypes.create_string_buffer(256)
    po, so = ctypes.c_int(-1), ctypes.c_int(-1)
    rc = lib.raw.fmha_fwd_hd128_mxfp8_auto(ctypes.byref(p), None, 0, None, ctypes.byref(po), ctypes.byref(so), err, 256)
    assert rc == code, (rc, err.value)


def test_auto_requires_workspace():
    """The KV-split path needs the caller's workspace of fmha_mxfp8_workspace_bytes (no allocation in the library)."""
    p = _params(path=2, splits=4, SK=4096)
    err = ctypes.create_string_buffer(256)
    po, so = ctypes.c_int(-1), ctypes.c_int(-1)
    rc = lib.raw.fmha_fwd_hd128_mxfp8_auto(ctypes.byref(p), None, 10, None, ctypes.byref(po), ctypes.byref(so), err, 256)
    assert rc == lib.FMHA_ERR_WORKSPACE, (rc, err.value)


def test_init_without_gpu_reports_error():
    """With no device the library reports FMHA_ERR_NO_DEVICE / FMHA_ERR_HIP instead of crashing."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    err = ctypes.create_string_buffer(256)
    rc = lib.raw.fmha_mxfp8_init(err, 256)
    assert rc in (lib.FMHA_ERR_NO_DEVICE, lib.FMHA_ERR_HIP) and err.value


def _f32_bits(x):
    return struct.unpack("<I", struct.pack("<f", x))[0]


def test_validate_scale_flag():
    """The in-kernel softmax scale (extension, flags bit 2 / kvs_splits bit 18) reads the f32 at 0x050, which the
    reference's MX kernels ignore: c = scale log2(e) must be a positive normal f32. Without the flag 0x050 is not
    checked (the reference's hosts write 1/sqrt(128) there)."""
    B, H, HK, S, SK = 2, 8, 4, 300, 1000
    a, sz = _shape_args(B, H, HK, S, SK)
    grid = (math.ceil(S / 256), H, B)
    a.softmax_scale = _f32_bits(float("nan"))
    assert lib.validate("vs128", a, sz, grid, HK=HK) == (0, "")
    a.flags = lib.FLAG_SCALE
    for bad in (0.0, -0.125, float("inf"), float("nan"), 1e-39, 3e38):
        a.softmax_scale = _f32_bits(bad)
        rc, msg = lib.validate("vs128", a, sz, grid, HK=HK)
        assert rc == lib.FMHA_ERR_KA_RANGE and "0x50" in msg, (bad, rc, msg)
    for good in (0.08838834764831845, 1.0, 2.0 ** -20, 1e4):
        a.softmax_scale = _f32_bits(good)
        assert lib.validate("vs128", a, sz, grid, HK=HK) == (0, ""), good
        assert lib.validate("t128", a, sz, (math.ceil(S / 128), H, B), HK=HK) == (0, ""), good
    ka, ksz, g = _kvsplit()
    set_scale = lambda x: ctypes.memmove(ctypes.addressof(ka) + 0x50, struct.pack("<f", x), 4)   # the base layout is raw bytes
    set_scale(0.0)
    assert lib.validate("kvsplit", ka, ksz, g, B=1, HK=8, KL=0) == (0, "")
    ka.kvs_splits = 8 | lib.KVS_SCALE
    assert lib.validate("kvsplit", ka, ksz, g, B=1, HK=8)[0] == lib.FMHA_ERR_KA_RANGE
    set_scale(0.5)
    assert lib.validate("kvsplit", ka, ksz, g, B=1, HK=8, KL=0) == (0, "")


def test_code_objects_have_no_calls():
    """Every kernel is one function: an outlined callee gets no kernel-argument pointer (it is not an ABI input) and
    reads its arguments from address 0. A code object with a call must not exist (build.py refuses to produce one)."""
    from amdgpu_rustdsl_amd import build
    for name in ("fmha_mxfp8_gfx950.hsaco", "mxfp8_quant_gfx950.hsaco"):
        path = os.path.join(os.path.dirname(lib.LIB_PATH), name)
        if not os.path.exists(path):
            pytest.skip(f"{name} not built")
        assert build.code_object_calls(path) == [], name


def test_op_signature_accepts_reference_kwargs():
    """A caller of the reference op (python/amdgpu_jit/ops.py:88) passes path, splits, specialize, stream and check by
    keyword; the op takes them with the same defaults."""
    import inspect
    from amdgpu_rustdsl_amd import ops
    sig = inspect.signature(ops.fmha_fwd_mxfp8)
    want = {"path": "auto", "splits": None, "specialize": True, "stream": None, "check": True}
    for name, default in want.items():
        assert sig.parameters[name].default == default, name
        assert sig.parameters[name].kind == inspect.Parameter.KEYWORD_ONLY, name
    assert list(sig.parameters)[:7] == ["q", "k", "v", "q_scale", "k_scale", "v_scale", "out"]


def test_no_check_skips_validate():
    """params.no_check (the op's check=False) skips the validate rules: a too-small output buffer is an extent error
    with the check and goes on to the launch without it (which, with no GPU here, reports the missing device)."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("the unchecked call would launch on the GPU")
    err = ctypes.create_string_buffer(256)
    po, so = ctypes.c_int(-1), ctypes.c_int(-1)
    p = _params(path=0)
    p.bytes_o = 16
    rc = lib.raw.fmha_fwd_hd128_mxfp8_auto(ctypes.byref(p), None, 0, None, ctypes.byref(po), ctypes.byref(so), err, 256)
    assert rc == lib.FMHA_ERR_EXTENT and b"GV-HOST-EXTENT" in err.value, (rc, err.value)
    p.no_check = 1
    rc = lib.raw.fmha_fwd_hd128_mxfp8_auto(ctypes.byref(p), None, 0, None, ctypes.byref(po), ctypes.byref(so), err, 256)
    assert rc in (lib.FMHA_ERR_NO_DEVICE, lib.FMHA_ERR_HIP), (rc, err.value)


def test_noalloc_rejects_oversized_split_before_gpu_work():
    """fmha_fwd_hd128_mxfp8_auto_noalloc refuses a split whose workspace exceeds its scratch array (the largest the
    auto dispatch asks for) before touching the device."""
    assert lib.NOALLOC_SCRATCH_BYTES == 2 * 32768 * 516 == max(
        lib.workspace_bytes(B, H, S, 2) for B, H, S in ((1, 8, 4096), (2, 16, 1024), (1, 1, 32768)))
    p = _params(path=2, splits=8, S=2048, SK=2048)
    err = ctypes.create_string_buffer(256)
    po, so = ctypes.c_int(-1), ctypes.c_int(-1)
    rc = lib.raw.fmha_fwd_hd128_mxfp8_auto_noalloc(ctypes.byref(p), None, ctypes.byref(po), ctypes.byref(so), err, 256)
    assert rc == lib.FMHA_ERR_WORKSPACE and b"GV-HOST-WORKSPACE" in err.value, (rc, err.value)



def test_causal_pair_flag_rules():
    """FMHA_FLAG_CAUSAL_PAIR (extension): only with the causal flag, only on the 128-row grid (t128 rules; the 256-row
    vs128 kernel refuses it), and the grid's x extent is then ceil(ceil(S / 128) / 2)."""
    B, H, S, SK = 2, 4, 1000, 1000
    a = lib.fill_args(0x1000, 0x2000, 0x3000, 0x4000, 0x5000, 0x6000, 0x7000, B, H, H, S, SK)
    big = 1 << 40
    sz = lib.BufferSizes(big, big, big, big, big, big, big, 0, 0)
    a.flags = lib.FLAG_CAUSAL | lib.FLAG_CAUSAL_PAIR
    assert lib.validate("t128", a, sz, (4, H, B), HK=H) == (0, "")           # T = 8 -> 4 blocks
    assert lib.validate("t128", a, sz, (8, H, B), HK=H)[0] == lib.FMHA_ERR_GRID
    assert lib.validate("vs128", a, sz, (2, H, B), HK=H)[0] == lib.FMHA_ERR_KA_RANGE
    a.flags = lib.FLAG_CAUSAL_PAIR
    assert lib.validate("t128", a, sz, (4, H, B), HK=H)[0] == lib.FMHA_ERR_KA_RANGE
    a.flags = lib.FLAG_CAUSAL | lib.FLAG_CAUSAL_PAIR
    a.s_seq_len, a.s_Bs, a.s_o_Bs, a.s_descale_q_Bs = 1152, 1152 * H * 128, 1152 * H * 256, 1152 * H * 4   # T = 9
    assert lib.validate("t128", a, sz, (5, H, B), HK=H) == (0, "")
    # causal full-sequence shapes run on the 128-row split-tile kernel (where the pairing is), from 4 key tiles on
    assert lib.uses_split_tiles("vs128", 4, 8, 2048, 2048, causal=True)
    assert not lib.uses_split_tiles("vs128", 4, 8, 2048, 2048, causal=False)
    assert not lib.uses_split_tiles("vs128", 4, 8, 2048, 384, causal=True)


@pytest.mark.parametrize("shape,chunks,parts", [
    ((1, 8, 128, 16384), 8, 32),     # config 5: 8 blocks per chunk -> 64, spread 4 ways -> 256 blocks of 4 key tiles
    ((1, 8, 128, 16000), 8, 16),     # 125 key tiles: 32 ranges would leave fewer than 4 tiles each
    ((1, 8, 128, 16384), 4, 32),     # the dispatch's 4 chunks: spread 8 ways (the most)
    ((1, 8, 2048, 2048), 4, 4),      # 256 blocks already
    ((1, 8, 512, 32768), 4, 16),     # 64 blocks -> 256
    ((1, 8, 512, 4096), 4, 8),       # 32 key tiles: 8 ranges of 4
    ((1, 8, 64, 1000), 2, 2),        # 8 key tiles: 2 ranges of 4 already
    ((1, 8, 2048, 2048), 8, 8),      # 512 blocks: beyond the CUs, no spread
    ((0, 8, 128, 4096), 4, 0),       # invalid sizes
])
def test_kv_partials_rule(shape, chunks, parts):
    """fmha_mxfp8_kv_partials (extension): chunks x sub, sub = 1, 2, 4 or 8 doubling while (S + 255) / 256 H B chunks
    sub blocks stay within the CU count (256 on MI355X; the value the library assumes without a device) and every
    key range keeps at least 4 key tiles."""
    assert lib.kv_partials(*shape, chunks) == parts


def test_workspace_turn_is_the_callers():
    """The KV split's workspace slot comes from the caller's own turn word (params.ws_turn), incremented once per call
    that reaches the slot choice: two threads with their own words and workspaces see exactly their own calls, in
    order, whatever the other does; no word (NULL) is slot 0 and leaves nothing behind. Runs without a GPU: the call
    then fails at the launch, after the slot choice."""
    import threading
    import torch
    if torch.cuda.is_available():
        pytest.skip("the calls would launch on the GPU")
    n = 200
    need = lib.workspace_bytes(1, 8, 128, lib.kv_partials(1, 8, 128, 4096, 4))
    words = [ctypes.c_uint32(0), ctypes.c_uint32(1000)]
    codes = [set(), set()]

    def worker(i):
        p = _params(path=2, splits=4, SK=4096)
        p.ws_turn = ctypes.pointer(words[i])
        err = ctypes.create_string_buffer(256)
        po, so = ctypes.c_int(-1), ctypes.c_int(-1)
        for _ in range(n):
            codes[i].add(lib.raw.fmha_fwd_hd128_mxfp8_auto(ctypes.byref(p), 0x10000 * (i + 1), 4 * need + 1024, None,
                                                           ctypes.byref(po), ctypes.byref(so), err, 256))
    ts = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert words[0].value == n and words[1].value == 1000 + n
    assert codes[0] <= {lib.FMHA_ERR_NO_DEVICE, lib.FMHA_ERR_HIP} and codes[1] <= {lib.FMHA_ERR_NO_DEVICE, lib.FMHA_ERR_HIP}
    # one slot's worth of workspace: no turn taken
    p = _params(path=2, splits=4, SK=4096)
    w = ctypes.c_uint32(7)
    p.ws_turn = ctypes.pointer(w)
    err = ctypes.create_string_buffer(256)
    po, so = ctypes.c_int(-1), ctypes.c_int(-1)
    lib.raw.fmha_fwd_hd128_mxfp8_auto(ctypes.byref(p), 0x10000, need, None, ctypes.byref(po), ctypes.byref(so), err, 256)
    assert w.value == 7


def test_auto_reports_chunks_and_partials():
    """*splits_out is the KV split's chunk count (the reference op's return value, python/amdgpu_jit/ops.py:143);
    params.partials_out receives the partials per row that run (chunks x the KV fill). Checked without a GPU: both are
    written before the launch."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("the call would launch on the GPU")
    for kv_fill, parts in ((0, 32), (1, 8)):
        p = _params(path=2, splits=8, S=128, SK=16384, kv_fill=kv_fill)
        got = ctypes.c_int32(-1)
        p.partials_out = ctypes.pointer(got)
        err = ctypes.create_string_buffer(256)
        po, so = ctypes.c_int(-1), ctypes.c_int(-1)
        need = lib.workspace_bytes(1, 8, 128, parts)
        rc = lib.raw.fmha_fwd_hd128_mxfp8_auto(ctypes.byref(p), 0x10000, need, None, ctypes.byref(po), ctypes.byref(so), err, 256)
        assert rc in (lib.FMHA_ERR_NO_DEVICE, lib.FMHA_ERR_HIP), (rc, err.value)
        assert (po.value, so.value, got.value) == (lib.PATH_KVSPLIT, 8, parts)
    # a full-sequence path: no split, no partials
    p = _params(path=0)
    got = ctypes.c_int32(-1)
    p.partials_out = ctypes.pointer(got)
    lib.raw.fmha_fwd_hd128_mxfp8_auto(ctypes.byref(p), None, 0, None, ctypes.byref(po), ctypes.byref(so), err, 256)
    assert (so.value, got.value) == (0, 0)


def test_unchecked_split_keeps_the_32bit_guard():
    """params.no_check skips the buffer-extent rules, not the kernel contract's 32-bit partial offsets: a split whose
    partials reach 4 GiB is refused either way."""
    for no_check in (0, 1):
        p = _params(path=2, splits=8, B=8, H=16, S=8192, SK=8192, kv_fill=1)   # 8 x 1 Mi rows x 512 B = 4 GiB
        p.no_check = no_check
        err = ctypes.create_string_buffer(256)
        po, so = ctypes.c_int(-1), ctypes.c_int(-1)
        rc = lib.raw.fmha_fwd_hd128_mxfp8_auto(ctypes.byref(p), 0x10000, 1 << 40, None, ctypes.byref(po), ctypes.byref(so), err, 256)
        assert rc == lib.FMHA_ERR_KA_RANGE and b"4 GiB" in err.value, (no_check, rc, err.value)


_CU_RULES = r"""
import json, sys
sys.path.insert(0, {root!r})
from amdgpu_rustdsl_amd import lib
print(json.dumps({{
    "parts": [lib.kv_partials(1, 8, 128, 16384, 8), lib.kv_partials(1, 8, 512, 32768, 4), lib.kv_partials(1, 8, 2048, 2048, 4)],
    "st": [lib.uses_split_tiles("vs128", 2, 8, 1024, 1024, causal=True), lib.uses_split_tiles("t128", 16, 8, 512, 512, causal=True)],
}}))
"""


@pytest.mark.parametrize("cus,parts,st", [
    # KV fill: blocks (S + 255) / 256 H B chunks, doubled while within the count and >= 4 key tiles per range;
    # causal split tiles: refused for <= 8 key tiles when the 128-row grid ((S + 127) / 128 H B) exceeds the count
    (None, [32, 16, 4], [True, False]),   # no device: 256, MI355X's count
    ("256", [32, 16, 4], [True, False]),
    ("304", [32, 16, 4], [True, False]),
    ("128", [16, 8, 4], [True, False]),
    ("80", [8, 4, 4], [False, False]),
    ("1024", [32, 32, 4], [True, True]),
])
def test_cu_dependent_rules(cus, parts, st):
    """The rules that follow the device's CU count (the KV fill, the causal split-tile choice), under
    FMHA_MXFP8_CU_COUNT: the output bits of those paths follow the count, so other parts get other (equally checked)
    orders."""
    import json
    import subprocess
    import sys
    env = dict(os.environ)
    env.pop("FMHA_MXFP8_CU_COUNT", None)
    if cus:
        env["FMHA_MXFP8_CU_COUNT"] = cus
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    out = subprocess.run([sys.executable, "-c", _CU_RULES.format(root=root)], env=env, capture_output=True, text=True,
                         check=True).stdout
    got = json.loads(out.strip().splitlines()[-1])
    assert got == {"parts": parts, "st": st}


def test_code_objects_keep_m0_to_the_copies():
    """M0 is written only by the kernels' own direct-copy sequences, and nothing the compiler emitted reads it
    (build.py refuses other code objects)."""
    from amdgpu_rustdsl_amd import build
    path = os.path.join(os.path.dirname(lib.LIB_PATH), "fmha_mxfp8_gfx950.hsaco")
    if not os.path.exists(path):
        pytest.skip("not built")
    assert build.code_object_m0_misuse(path) == []
