"""Build of the native library: the gfx950 code object and the C-ABI host library that embeds it.

    python amdgpu_rustdsl_amd/build.py         # or __graft_entry__.build()

Outputs (in-tree, git-ignored, shipped with the source tree):
    amdgpu_rustdsl_amd/_build/fmha_mxfp8_gfx950.hsaco   the four FMHA kernels (hipcc --genco, gfx950 only)
    amdgpu_rustdsl_amd/_build/mxfp8_quant_gfx950.hsaco  the quantisers
    amdgpu_rustdsl_amd/_build/libfmha_mxfp8.so          include/fmha_mxfp8.h + include/mxfp8_quant.h, both code
                                                        objects embedded
"""
import os
import subprocess
import tempfile
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
OUT = os.path.join(PKG, "_build")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HSACO = os.path.join(OUT, "fmha_mxfp8_gfx950.hsaco")
QHSACO = os.path.join(OUT, "mxfp8_quant_gfx950.hsaco")
LIB = os.path.join(OUT, "libfmha_mxfp8.so")

# Packed FP32 VALU forms are kept out of the kernels (their results have been unreliable on this hardware pool);
# the host pass warns that it does not know the feature, which is harmless.
HIP_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wno-unused-command-line-argument"]
# The attention kernels: MFMA accumulators and sources in the VGPR form. The 256-thread t128 kernel needs more than
# 256 registers per wave; left to choose, the compiler placed the QK MFMAs' S accumulators in AGPRs and moved all 64
# back to VGPRs for the softmax every tile (80 v_accvgpr moves per tile in the loop). In the VGPR form other values
# take the AGPRs and the loop has none. The other kernels fit in 256 VGPRs and compile to the same code either way.
# Kernel-argument preload: the first 9 dwords of scalar kernel parameters arrive in SGPRs at wave launch (the combines,
# whose 36-byte layout is nine dwords of scalars); the attention kernels take one aggregate parameter, which is not
# preloaded, and compile to the same code with or without it.
FMHA_FLAGS = ["-mllvm", "-amdgpu-mfma-vgpr-form", "-mllvm", "-amdgpu-kernarg-preload-count=9"]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("build step failed: " + " ".join(cmd))
    return r


def code_object_calls(hsaco):
    """Call instructions in the gfx950 code object inside a --genco bundle (the kernels must be one function each:
    in an outlined callee the kernel-argument pointer is not an ABI input and compiles to null, so its first
    argument read faults). Returns the offending lines."""
    llvm = os.path.join(ROCM, "llvm", "bin")
    with tempfile.TemporaryDirectory() as td:
        co = os.path.join(td, "k.co")
        _run([os.path.join(llvm, "clang-offload-bundler"), "--unbundle", "--type=o", "--input=" + hsaco,
              "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", "--output=" + co])
        dis = _run([os.path.join(llvm, "llvm-objdump"), "-d", "--no-show-raw-insn", co]).stdout
    return [l.strip() for l in dis.splitlines() if "s_swappc_b64" in l or "s_call_b64" in l]


# Instructions that read M0 implicitly (gfx950). The direct HBM -> LDS copies of the attention kernels set M0 in inline
# assembly; a compiler-emitted reader would see their value.
_M0_READERS = ("s_sendmsg", "ds_gws", "ds_append", "ds_consume", "ds_read_addtid", "ds_write_addtid", "s_movrel",
               "v_movrel", "v_interp", "lds_param_load", "lds_direct_load", "global_load_lds", "s_ttracedata")


def code_object_m0_misuse(hsaco):
    """M0 in the gfx950 code object: every write must be the copy sequence `s_mov_b32 m0, sN; s_nop 0;
    buffer_load_* ... lds` of the kernels' inline assembly, and no other instruction may read or write M0. Returns
    the offending lines."""
    llvm = os.path.join(ROCM, "llvm", "bin")
    with tempfile.TemporaryDirectory() as td:
        co = os.path.join(td, "k.co")
        _run([os.path.join(llvm, "clang-offload-bundler"), "--unbundle", "--type=o", "--input=" + hsaco,
              "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", "--output=" + co])
        dis = _run([os.path.join(llvm, "llvm-objdump"), "-d", "--no-show-raw-insn", co]).stdout
    ins = [l.split("//")[0].strip() for l in dis.splitlines()]
    ins = [l for l in ins if l and not l.endswith(":") and not l.startswith("Disassembly") and " file format" not in l]
    bad = []
    for i, l in enumerate(ins):
        op = l.split()[0]
        if op.startswith(_M0_READERS):
            bad.append(l)
        elif "m0" in l.replace(",", " ").split()[1:]:
            ok = (op == "s_mov_b32" and l.split()[1].rstrip(",") == "m0" and i + 2 < len(ins)
                  and ins[i + 1].split()[0] == "s_nop" and ins[i + 2].startswith("buffer_load_") and ins[i + 2].endswith(" lds"))
            if not ok:
                bad.append(l)
        elif op.startswith("buffer_load_") and l.endswith(" lds"):
            if not (i >= 2 and ins[i - 2].startswith("s_mov_b32 m0,")):
                bad.append(l)
    return bad


def build(verbose=False):
    os.makedirs(OUT, exist_ok=True)
    hipcc = os.path.join(ROCM, "bin", "hipcc")
    _run([hipcc, *HIP_FLAGS, *FMHA_FLAGS, "--genco", os.path.join(CSRC, "fmha_kernels.hip"), "-o", HSACO])
    _run([hipcc, *HIP_FLAGS, "--genco", os.path.join(CSRC, "quant_kernels.hip"), "-o", QHSACO])
    for co in (HSACO, QHSACO):
        calls = code_object_calls(co)
        if calls:
            os.remove(co)
            raise RuntimeError(f"{co}: a kernel calls an outlined function ({calls[0]}); force-inline it")
        m0 = code_object_m0_misuse(co)
        if m0:
            os.remove(co)
            raise RuntimeError(f"{co}: M0 used outside the kernels' copy sequences ({m0[0]})")
    # the allocation-free entry is single-source HIP (its device array is registered with the runtime at load time)
    noalloc_o = os.path.join(OUT, "fmha_noalloc.o")
    _run([hipcc, *HIP_FLAGS, "-fPIC", "-c", os.path.join(CSRC, "fmha_noalloc.hip"), "-o", noalloc_o])
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wextra", "-D__HIP_PLATFORM_AMD__",
          "-I" + os.path.join(ROCM, "include"), '-DFMHA_HSACO_PATH="%s"' % HSACO, '-DMXQ_HSACO_PATH="%s"' % QHSACO,
          os.path.join(CSRC, "fmha_host.cpp"), os.path.join(CSRC, "quant_host.cpp"), noalloc_o, "-L" + os.path.join(ROCM, "lib"), "-lamdhip64",
          "-Wl,-rpath," + os.path.join(ROCM, "lib"), "-o", LIB])
    if verbose:
        print("built", HSACO, os.path.getsize(HSACO), "bytes;", LIB, os.path.getsize(LIB), "bytes")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
