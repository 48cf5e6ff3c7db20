"""Build recipe for the gfx950 HIP library ``libmindpipe_amd.so`` (in-tree).

``python -m mindpipe_amd.build`` compiles every ``csrc/*.hip`` with hipcc for
gfx950 and links the C-ABI shared library next to this file.  The library
exports exactly the ``extern "C"`` functions declared in
``include/mindpipe_amd.h``.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "libmindpipe_amd.so"
BUILD_DIR = PKG / "_build"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # packed fp32 VALU ops (v_pk_{add,mul,fma}_f32) stay off: some of their forms have given
    # wrong results on this hardware without an error
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


# Per-source extra flags.  w4a16.hip: MFMA results in ordinary VGPRs (its
# kernels scale every MFMA result in VALU code; results in accumulation registers
# would each need a copy first).
FILE_FLAGS = {
    "w4a16.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


# ``--knobs`` (or MINDPIPE_AMD_KNOBS=1) builds a measurement library whose kernel choice follows
# the MP_W4_* / MP_W8_* environment variables; the default library ignores them.
KNOB_FLAGS = ["-DMP_MEASUREMENT_KNOBS"]


def _knobs() -> bool:
    return "--knobs" in sys.argv[1:] or os.environ.get("MINDPIPE_AMD_KNOBS") == "1"


def _compile(src: Path) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [HIPCC, *FLAGS, *(KNOB_FLAGS if _knobs() else []), *FILE_FLAGS.get(src.name, []), "-c", str(src),
           "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")
    noise = "is not a recognized feature for this target"
    msgs = [l for l in (res.stderr or "").splitlines() if l.strip() and noise not in l]
    if msgs:
        print("\n".join(msgs), file=sys.stderr)
    return obj


def _stale(src: Path) -> bool:
    """An object is stale when it is missing or older than its source or any shared header."""
    obj = BUILD_DIR / (src.stem + ".o")
    if not obj.exists():
        return True
    deps = [src, *CSRC.glob("*.h"), PKG.parent / "include" / "mindpipe_amd.h", Path(__file__)]
    return any(d.stat().st_mtime > obj.stat().st_mtime for d in deps if d.exists())


MEASURE_DIR = PKG / "measure"
MEASURE_LIB = MEASURE_DIR / "libmindpipe_measure.so"


def build_measure(verbose: bool = True) -> Path:
    """The measurement-only probe library (``measure/probe.hip``), outside the product ABI."""
    src = MEASURE_DIR / "probe.hip"
    tmp = MEASURE_LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, *FLAGS, "-shared", str(src), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, MEASURE_LIB)
    if verbose:
        print(f"built {MEASURE_LIB}")
    return MEASURE_LIB


def build(verbose: bool = True, incremental: bool = False) -> Path:
    """Compile every ``csrc/*.hip`` and link the library.  ``incremental=True`` (a development
    aid) recompiles only sources whose object is stale."""
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    BUILD_DIR.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    todo = [s for s in srcs if _stale(s)] if incremental else srcs
    with cf.ThreadPoolExecutor(max_workers=max(1, min(8, len(todo)))) as ex:
        list(ex.map(_compile, todo))
    objs = [BUILD_DIR / (s.stem + ".o") for s in srcs]
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {[s.name for s in srcs]}")
    if not incremental or not MEASURE_LIB.exists() or \
            (MEASURE_DIR / "probe.hip").stat().st_mtime > MEASURE_LIB.stat().st_mtime:
        build_measure(verbose)
    return LIB


if __name__ == "__main__":
    build(incremental="--incremental" in sys.argv[1:])
