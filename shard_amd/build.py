"""Build libshard_hip.so (gfx950) in-tree with hipcc.

    python -m shard_amd.build            # or shard_amd.build.build()

Each ``csrc/*.hip`` is compiled to an object with its own flags (the integer
chains in quant.hip with -ffp-contract=off so no multiply-add is fused), then
all objects are linked into ``shard_amd/libshard_hip.so``.
"""
import os
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libshard_hip.so")
ARCH = os.environ.get("SHARD_OFFLOAD_ARCH", "gfx950")

COMMON = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    # packed fp32 arithmetic stays off in all device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]
PER_FILE = {
    "quant.hip": ["-ffp-contract=off"],
    "decode_attn.hip": [],
    "pca.hip": ["-ffp-contract=off"],  # the fused undo-RoPE rounds as k_prepare does
    "reconstruct.hip": ["-ffp-contract=off"],
    "abi.hip": [],
    "fp16_decode.hip": [],
}


def hipcc() -> str:
    p = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(p):
        raise RuntimeError("hipcc not found; libshard_hip.so cannot be built")
    return p


def sources():
    return sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))


def build(verbose: bool = False, jobs: int = 4) -> str:
    """Compile every csrc/*.hip for gfx950 and link libshard_hip.so. Returns its path."""
    cc = hipcc()
    objdir = tempfile.mkdtemp(prefix="shard_build_")
    try:
        procs, objs = [], []
        for src in sources():
            obj = os.path.join(objdir, src.replace(".hip", ".o"))
            cmd = [cc, *COMMON, *PER_FILE.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
            if verbose:
                print(" ".join(cmd), flush=True)
            procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE,
                                                stderr=subprocess.STDOUT, text=True)))
            objs.append(obj)
            if len(procs) >= jobs:
                _drain(procs)
        _drain(procs)
        tmp = LIB + ".tmp"
        cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
        out = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
        if out.returncode != 0:
            raise RuntimeError("link failed:\n" + out.stdout)
        os.replace(tmp, LIB)
    finally:
        shutil.rmtree(objdir, ignore_errors=True)
    return LIB


def _drain(procs):
    while procs:
        src, p = procs.pop(0)
        out, _ = p.communicate()
        if p.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src}:\n{out}")
        warn = [ln for ln in out.splitlines() if "warning" in ln and "packed-fp32-ops" not in ln]
        if warn:
            sys.stderr.write(f"[{src}]\n" + "\n".join(warn[:20]) + "\n")


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
