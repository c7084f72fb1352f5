"""Builds hw_probe.hip (``--build``, on any machine with hipcc) and runs it on a gfx950 GPU (``--run OUT.npz``),
recording what the hardware conversion and MFMA instructions return on fixed inputs. The committed
``hw_probe.npz`` next to this script is the output of ``--run``; the CPU tests compare the oracle's restatements of
these instructions against it.

    python tests/golden/make_hw_fixture.py --build
    python tests/golden/make_hw_fixture.py --run /tmp/hw_probe.npz           (on a machine with a gfx950 GPU)
"""
import argparse
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
SO = os.path.join(HERE, "_build", "hw_probe.so")


def pknorm_inputs():
    """f32 inputs of the pknorm probe: the clamp edges, values next to every representable quarter step, and 60000
    seeded uniforms over [-0.25, 1.25]."""
    rng = np.random.default_rng(20261201)
    edge = np.array([-1e30, -1.0, -0.0, 0.0, 1e-30, 1.0, 1.0000001, 2.0, 1e30, np.inf, -np.inf], np.float32)
    k = np.arange(0, 65536, 16, dtype=np.float64)
    ties = ((k + 0.5) / 65535.0).astype(np.float32)      # near the rounding midpoints
    near = np.nextafter(ties, np.float32(2.0))
    u = rng.uniform(-0.25, 1.25, 60000).astype(np.float32)
    x = np.concatenate([edge, ties, near, u]).astype(np.float32)
    if x.size % 2:
        x = np.concatenate([x, np.float32([0.5])])
    return x


def mfma_inputs():
    """Operands of the scaled MFMA probe: e4m3 bytes (finite, no NaN 0x7F / 0xFF), scale bytes in [118, 136], C."""
    rng = np.random.default_rng(7)
    a = rng.integers(0, 256, (64, 32), dtype=np.uint8)
    b = rng.integers(0, 256, (64, 32), dtype=np.uint8)
    for t in (a, b):
        t[(t & 0x7F) == 0x7F] = 0x38
    sa = rng.integers(118, 137, 64).astype(np.int32)
    sb = rng.integers(118, 137, 64).astype(np.int32)
    c = rng.standard_normal((64, 16)).astype(np.float32)
    return a, b, sa, sb, c


def build():
    os.makedirs(os.path.dirname(SO), exist_ok=True)
    subprocess.run(["hipcc", "--offload-arch=gfx950", "-O2", "-shared", "-fPIC", "-Xclang", "-target-feature", "-Xclang",
                    "-packed-fp32-ops", os.path.join(HERE, "hw_probe.hip"), "-o", SO], check=True)


def run(out):
    lib = ctypes.CDLL(SO)
    x = pknorm_inputs()
    a, b, sa, sb, c = mfma_inputs()
    cvt = np.zeros(131072, np.uint8)
    pk = np.zeros(x.size, np.uint16)
    d = np.zeros((64, 16), np.float32)
    P = lambda t: t.ctypes.data_as(ctypes.c_void_p)
    rc = lib.hw_probe_run(P(cvt), P(x), P(pk), ctypes.c_uint32(x.size), P(np.ascontiguousarray(a)), P(np.ascontiguousarray(b)),
                          P(sa), P(sb), P(c), P(d))
    if rc:
        raise SystemExit(f"hw_probe_run failed: {rc}")
    np.savez_compressed(out, cvt=cvt.reshape(2, 65536), pk_in=x, pk_out=pk, mfma_a=a, mfma_b=b, mfma_sa=sa, mfma_sb=sb,
                        mfma_c=c, mfma_d=d)
    print("wrote", out)


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--build", action="store_true")
    ap.add_argument("--run", metavar="OUT")
    args = ap.parse_args()
    if args.build:
        build()
    if args.run:
        run(args.run)
