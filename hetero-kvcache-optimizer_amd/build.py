"""Build libheterokv.so (HIP, gfx950) in-tree.

    python hetero-kvcache-optimizer_amd/build.py

Compiles every csrc/*.hip file with hipcc for gfx950 into
heterokv/libheterokv.so.  Correctly rounded fp32 division/sqrt stay on (the
quantizer is bit-exact with an IEEE reference) and packed-fp32 instructions are
disabled for device code.  The streaming-read probes (csrc/probe/*.hip, used by
bench.py's probe workload only) go into heterokv/libhkvprobe.so.
"""
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
OUT = os.path.join(PKG_DIR, "heterokv", "libheterokv.so")
PROBE_OUT = os.path.join(PKG_DIR, "heterokv", "libhkvprobe.so")

HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    "--offload-arch=gfx950",
    "-fPIC",
    "-shared",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-fast-math",
    "-ffp-contract=on",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # The AMDGPU atomic optimizer turns a single-lane atomic whose result is used later
    # (the decode kernel's placement-mask OR) into a wave-aggregated one that waits for
    # the result at once, which puts an L2 round trip in front of the workgroup merge.
    # Every other atomic in the library is a single-lane error-bit OR on a rare path.
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
    "-Wno-unused-command-line-argument",
]


def hipcc_path():
    p = shutil.which("hipcc")
    if p is None and os.path.exists("/opt/rocm/bin/hipcc"):
        p = "/opt/rocm/bin/hipcc"
    if p is None:
        raise RuntimeError("hipcc not found: the HIP library cannot be built")
    return p


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(srcs, out_path, verbose):
    tmp = out_path + ".tmp"
    cmd = [hipcc_path()] + HIPCC_FLAGS + ["-o", tmp] + srcs
    if verbose:
        print("[heterokv] " + " ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = res.stdout
    # the host pass does not know the device-only feature name; that warning is expected
    lines = [ln for ln in out.splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
    if res.returncode != 0:
        sys.stderr.write(out)
        raise RuntimeError("hipcc failed with exit code %d" % res.returncode)
    if verbose and lines:
        print("\n".join(lines), flush=True)
    os.replace(tmp, out_path)


def build(verbose=True):
    _compile(sources(), OUT, verbose)
    probe_dir = os.path.join(CSRC, "probe")
    _compile(sorted(os.path.join(probe_dir, f) for f in os.listdir(probe_dir) if f.endswith(".hip")), PROBE_OUT,
             verbose)
    return OUT


if __name__ == "__main__":
    print(build())
