"""Build libnslg_kv.so (the C-ABI KV-cache library) for gfx950 with hipcc.

Each ``csrc/*.hip`` file is compiled to an object in ``csrc/_obj`` (in
parallel), then linked into ``nanoslg_amd/libnslg_kv.so``. The library links the
HIP runtime dynamically; loaded after ``import torch`` it binds to the runtime
torch already mapped, so the process holds a single HIP runtime.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
OBJ_DIR = CSRC / "_obj"
LIB_PATH = PKG_DIR / "libnslg_kv.so"
# the CPython fast-call binding of the per-step entry points (links libnslg_kv.so)
FAST_SRC = CSRC / "fastcall.c"
FAST_PATH = PKG_DIR / ("_nslg_fast" + (sysconfig.get_config_var("EXT_SUFFIX") or ".so"))
# the host-side forward planner (plain C over the CPython API, no GPU code)
HOST_SRC = CSRC / "host_plan.c"
HOST_PATH = PKG_DIR / ("_nslg_host" + (sysconfig.get_config_var("EXT_SUFFIX") or ".so"))
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-ffp-contract=fast",
    "-munsafe-fp-atomics",
    # Packed fp32 VALU ops stay disabled in all device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
    # keep MFMA accumulators in ordinary VGPRs (no per-tile AGPR copies)
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]


# Extra flags for single sources. The prefill kernel's softmax takes running maxima
# of scores that are never NaN for finite inputs; without NaN semantics the
# compiler drops the quieting copy it otherwise puts in front of every max.
FILE_FLAGS = {
    "paged_prefill.hip": ["-fno-honor-nans"],
}


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (looked in $HIPCC, /opt/rocm/bin, PATH)")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile_one(hipcc: str, src: Path, extra: list[str]) -> Path:
    obj = OBJ_DIR / (src.stem + ".o")
    cmd = [hipcc, *HIPCC_FLAGS, *FILE_FLAGS.get(src.name, []), *extra, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return obj


def build(verbose: bool = False, extra_flags: list[str] | None = None) -> Path:
    """Compile every HIP source and link the shared library. Always rebuilds."""
    hipcc = _hipcc()
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    extra = list(extra_flags or [])
    srcs = sources()
    workers = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(max_workers=workers) as ex:
        objs = list(ex.map(lambda s: _compile_one(hipcc, s, extra), srcs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    _build_fast()
    _build_host()
    if verbose:
        print(f"[nanoslg_amd] built {LIB_PATH} from {len(srcs)} sources, {FAST_PATH.name} and {HOST_PATH.name}",
              file=sys.stderr)
    return LIB_PATH


def _cc() -> str:
    cc = os.environ.get("CC") or shutil.which("gcc") or shutil.which("cc")
    if not cc:
        raise RuntimeError("no C compiler (gcc) for the CPython extensions")
    return cc


def _build_ext(src: Path, out: Path, link: list[str]) -> None:
    tmp = out.with_suffix(".so.tmp")
    cmd = [_cc(), "-O2", "-shared", "-fPIC", "-Wall", "-Wno-unused-parameter",
           f"-I{sysconfig.get_paths()['include']}", str(src), "-o", str(tmp), *link]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"{src.name} failed:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)


def _build_fast() -> None:
    """Compile the fast-call binding (host C, the system compiler) against the
    library just linked; it finds the library next to itself at run time."""
    _build_ext(FAST_SRC, FAST_PATH, [f"-L{PKG_DIR}", "-lnslg_kv", "-Wl,-rpath,$ORIGIN"])


def _build_host() -> None:
    """Compile the host-side forward planner (host C, no library to link)."""
    _build_ext(HOST_SRC, HOST_PATH, [])


if __name__ == "__main__":
    build(verbose=True)
