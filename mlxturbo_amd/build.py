"""Build ``libmlxturbo_amd.so`` in-tree with hipcc for gfx950.

Usage: ``python -m mlxturbo_amd.build``.  The library is plain C ABI over HIP
(no torch headers): ``csrc/abi.hip`` (argument checks and routing) plus
``csrc/inst.hip`` compiled once per (dtype, bits) pair, in parallel, then
linked into one shared object.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libmlxturbo_amd.so")
# measurement helper for bench.py (a plain streaming read), not part of the ABI
PROBE_SRC = os.path.join(CSRC, "read_probe.hip")
PROBE_OUT = os.path.join(HERE, "libmq_read_probe.so")
ARCH = os.environ.get("MQ_OFFLOAD_ARCH", "gfx950")

# -packed-fp32-ops: never emit v_pk_{add,mul,fma}_f32 (hipcc's host pass warns
# that it does not know the feature; that is harmless).
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm required to build mlxturbo_amd)")


# (source, extra defines) of each translation unit
UNITS = [("abi.hip", []), ("formats.hip", []), ("prep.hip", []), ("route.hip", []),
         ("swiglu.hip", [])] + [
    ("inst.hip", [f"-DMQ_INST_DT={dt}", f"-DMQ_INST_BITS={bits}"] + glu)
    for glu in ([], ["-DMQ_INST_GLU"]) for dt in (0, 1) for bits in (4, 8)
] + [
    # the quad kernel keeps its MFMA accumulators in VGPRs (qmv_quad.cuh)
    ("quad.hip", [f"-DMQ_INST_DT={dt}", f"-DMQ_INST_BITS={bits}", "-mllvm",
                  "-amdgpu-mfma-vgpr-form"])
    for dt in (0, 1) for bits in (4, 8)
]

_NOISE = ("packed-fp32-ops", "warning generated", "warnings generated")


def sources() -> list[str]:
    return sorted({os.path.join(CSRC, src) for src, _ in UNITS})


def _filtered(stderr: str) -> str:
    return "\n".join(l for l in stderr.splitlines() if not any(n in l for n in _NOISE))


def build(verbose: bool = False) -> str:
    compile_flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    with tempfile.TemporaryDirectory(prefix="mq_build_") as tmpdir:
        probe_cmd = [hipcc(), *HIPCC_FLAGS, "-o", PROBE_OUT + ".tmp", PROBE_SRC]
        if verbose:
            print(" ".join(probe_cmd), flush=True)
        probe = subprocess.Popen(probe_cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE,
                                 text=True)
        procs = []
        for i, (src, defs) in enumerate(UNITS):
            obj = os.path.join(tmpdir, f"unit{i}.o")
            cmd = [hipcc(), *compile_flags, *defs, "-c", "-o", obj, os.path.join(CSRC, src)]
            if verbose:
                print(" ".join(cmd), flush=True)
            procs.append((obj, cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE,
                                                     stderr=subprocess.PIPE, text=True)))
        objs = []
        failed = []
        for obj, cmd, proc in procs:
            _, err = proc.communicate()
            if proc.returncode != 0:
                failed.append(f"{' '.join(cmd)}\n{_filtered(err)}")
            elif verbose and _filtered(err).strip():
                print(_filtered(err), file=sys.stderr)
            objs.append(obj)
        _, err = probe.communicate()
        if probe.returncode != 0:
            failed.append(f"{' '.join(probe_cmd)}\n{_filtered(err)}")
        if failed:
            raise RuntimeError("hipcc failed:\n" + "\n\n".join(failed))
        os.replace(PROBE_OUT + ".tmp", PROBE_OUT)
        tmp = OUT + ".tmp"
        cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"link failed ({res.returncode}):\n{_filtered(res.stderr)}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
