"""Build the MI355X MatMulNBits libraries in-tree.

Outputs (under ``lib/`` next to this file):

* ``libmnb_hip.so`` — the gfx950 HIP kernels plus the C-ABI shim (``include/mnb_hip.h``).
* ``libonnxruntime_mi355x_ep.so`` — the ONNX Runtime plugin EP (``include/onnxruntime_mi355x_ep.h``),
  linked against ``libmnb_hip.so`` with an ``$ORIGIN`` rpath.

Every HIP translation unit is compiled with ``--offload-arch=gfx950`` and with the packed-fp32
target feature switched off.  Objects are rebuilt only when a source or header is newer.
Run as ``python onnxruntime-ep-vulkan_amd/build.py [--force] [-j N]``.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "lib"
OBJ = PKG / "_build"
INCLUDE = REPO / "include"
# ORT's plugin-EP C headers (ONNX Runtime v1.28.0, MIT), vendored under third_party/onnxruntime
# (ORT_INCLUDE_DIR overrides them).
ORT_INCLUDE_CANDIDATES = [
    Path(os.environ.get("ORT_INCLUDE_DIR", "")),
    REPO / "third_party" / "onnxruntime" / "include",
]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
]
# MFMA results in architectural VGPRs, where the fp32 block epilogues read them, instead of AGPRs
# that need a v_accvgpr_read per element -- for every kernel but the calibration loop, whose
# sixteen accumulators are only ever read by MFMAs.
VGPR_MFMA = ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]

HIP_SOURCES = [
    CSRC / "kernels" / "mnb_gemv.hip",
    CSRC / "kernels" / "mnb_gemm.hip",
    CSRC / "kernels" / "mnb_group_gemv.hip",
    CSRC / "kernels" / "mnb_strip_gemv.hip",
    CSRC / "kernels" / "mnb_acc4_stream.hip",
    CSRC / "kernels" / "mnb_batch_stream.hip",
    CSRC / "kernels" / "mnb_gemv_stream.hip",
    CSRC / "kernels" / "mnb_gemv_stream_b4.hip",
    CSRC / "kernels" / "mnb_gemv_stream_b8.hip",
    CSRC / "kernels" / "mnb_gemv_f32.hip",
    CSRC / "kernels" / "mnb_gemm_f32.hip",
    CSRC / "kernels" / "mnb_calibrate.hip",
    CSRC / "kernels" / "mnb_qmoe.hip",
    CSRC / "kernels" / "mnb_rmsnorm.hip",
    CSRC / "kernels" / "mnb_gqa.hip",
    CSRC / "kernels" / "mnb_stage.hip",
    CSRC / "shim" / "mnb_shim.hip",
]
EP_SOURCES: list[Path] = sorted((CSRC / "ep").glob("*.cpp"))


def _headers() -> list[Path]:
    # build.py itself is a dependency: a change of flags rebuilds every object
    return list(CSRC.rglob("*.hpp")) + list(INCLUDE.glob("*.h")) + [Path(__file__)]


def _stale(out: Path, deps: list[Path]) -> bool:
    if not out.exists():
        return True
    t = out.stat().st_mtime
    return any(d.stat().st_mtime > t for d in deps if d.exists())


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + r.stdout + r.stderr)
        raise RuntimeError(f"build step failed: {cmd[0]} … {cmd[-1]}")


def _compile_hip(src: Path, force: bool) -> Path:
    obj = OBJ / (src.stem + ".o")
    if force or _stale(obj, [src] + _headers()):
        extra = [] if src.stem == "mnb_calibrate" else VGPR_MFMA
        _run([HIPCC, *HIP_FLAGS, *extra, "-c", str(src), "-o", str(obj)])
    return obj


def ort_include_dir() -> Path | None:
    for c in ORT_INCLUDE_CANDIDATES:
        if str(c) and (c / "onnxruntime_ep_c_api.h").exists():
            return c
    return None


def build(force: bool = False, jobs: int = 8) -> dict[str, Path]:
    LIB.mkdir(exist_ok=True)
    OBJ.mkdir(exist_ok=True)
    out: dict[str, Path] = {}
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile_hip(s, force), HIP_SOURCES))
    hip_lib = LIB / "libmnb_hip.so"
    if force or _stale(hip_lib, objs):
        _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(hip_lib),
              *map(str, objs), "-Wl,-soname,libmnb_hip.so"])
    out["hip"] = hip_lib

    if EP_SOURCES:
        ort_inc = ort_include_dir()
        if ort_inc is None:
            raise RuntimeError("ORT plugin-EP headers not found; set ORT_INCLUDE_DIR")
        ep_lib = LIB / "libonnxruntime_mi355x_ep.so"
        ep_objs = []
        for src in EP_SOURCES:
            obj = OBJ / (src.stem + ".ep.o")
            if force or _stale(obj, [src] + _headers()):
                _run(["g++", "-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra",
                      "-fvisibility=hidden", f"-I{INCLUDE}", f"-I{ort_inc}", f"-I{CSRC / 'ep'}",
                      "-c", str(src), "-o", str(obj)])
            ep_objs.append(obj)
        if force or _stale(ep_lib, ep_objs + [hip_lib]):
            _run(["g++", "-shared", "-fPIC", "-o", str(ep_lib), *map(str, ep_objs),
                  f"-L{LIB}", "-lmnb_hip", "-Wl,-rpath,$ORIGIN", "-Wl,--no-undefined",
                  "-Wl,-soname,libonnxruntime_mi355x_ep.so", "-pthread"])
        out["ep"] = ep_lib
    return out


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--force", action="store_true")
    ap.add_argument("-j", type=int, default=8)
    a = ap.parse_args()
    for k, v in build(force=a.force, jobs=a.j).items():
        print(f"{k}: {v}")


if __name__ == "__main__":
    main()
