"""Writes tests/golden/ref_inputs.json: SHA-256 digests of the inputs that the reference's own harness generates
(tests/gpu/ref_host.cpp:183-263, dumped by REF_INPUT_DUMP at :282-286) for the run_ref.sh shape list
(run_ref.sh:57), the determinism shapes (determinism.sh:56) and the BASELINE configs, in its three data modes.
tests/test_oracle.py::test_generator_matches_reference_harness checks the oracle's restatement (oracle.Inputs)
against them byte for byte.

Runs oracle/_ref/ref_host (built from the reference's source by oracle/Makefile.ref) on a machine with a GPU: the
harness copies its inputs to the device before dumping them, then fails to load the vendor code object it is given
(a path that does not exist) and exits; nothing else of it runs.

    python tests/golden/make_ref_inputs_fixture.py [out.json]
"""
import hashlib
import json
import os
import subprocess
import sys
import tempfile

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
REF_HOST = os.path.join(ROOT, "oracle", "_ref", "ref_host")

# (B, H, S, SK, gqa): run_ref.sh:57, then determinism.sh:56 (a subset of it), then BASELINE configs 1-5
SHAPES = [(1, 1, 256, 256, 1), (1, 2, 512, 512, 1), (2, 4, 1024, 1024, 1), (1, 8, 2048, 2048, 1), (1, 2, 512, 2048, 1),
          (3, 3, 768, 1280, 1), (1, 4, 300, 512, 1), (2, 8, 700, 640, 2), (1, 16, 256, 1024, 4), (1, 2, 256, 1000, 1),
          (2, 4, 300, 129, 1), (1, 8, 512, 100, 2), (1, 2, 1024, 1088, 1), (1, 4, 77, 1, 1), (1, 2, 200, 1337, 2),
          (4, 8, 2048, 2048, 1), (1, 8, 8192, 8192, 1), (2, 8, 2048, 2048, 1), (1, 8, 128, 16384, 1), (1, 8, 128, 16000, 1)]
MODES = ["lcg", "uniform", "normal"]


def main():
    out = sys.argv[1] if len(sys.argv) > 1 else os.path.join(ROOT, "tests", "golden", "ref_inputs.json")
    entries = []
    with tempfile.TemporaryDirectory() as td:
        for (B, H, S, SK, g) in SHAPES:
            for mode in MODES:
                if mode != "normal" and (B, H, S, SK) in ((4, 8, 2048, 2048), (1, 8, 8192, 8192)):
                    continue   # the large configs only in the published mode
                prefix = os.path.join(td, "in")
                env = dict(os.environ, REF_B=str(B), REF_H=str(H), REF_S=str(S), REF_SK=str(SK), REF_HK=str(H // g),
                           REF_DATA=mode, REF_INPUT_DUMP=prefix)
                r = subprocess.run([REF_HOST, os.path.join(td, "no_vendor.co")], env=env, capture_output=True, text=True,
                                   timeout=120)
                digests = {}
                for ext in ("q", "k", "v", "qs", "ks"):
                    with open(f"{prefix}.{ext}", "rb") as f:
                        data = f.read()
                    digests[ext] = {"bytes": len(data), "sha256": hashlib.sha256(data).hexdigest()}
                    os.remove(f"{prefix}.{ext}")
                print(f"B{B} H{H} S{S} SK{SK} gqa{g} {mode}: rc={r.returncode} {digests['q']['sha256'][:12]}", flush=True)
                entries.append({"B": B, "H": H, "S": S, "SK": SK, "gqa": g, "mode": mode, "digests": digests})
    with open(out, "w") as f:
        json.dump({"source": "tests/gpu/ref_host.cpp (REF_INPUT_DUMP), built by oracle/Makefile.ref", "entries": entries}, f,
                  indent=1)
    print("wrote", out)


if __name__ == "__main__":
    main()
