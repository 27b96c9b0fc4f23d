"""In-tree build of the gfx950 library and its PyTorch host extension.

Produces, next to this file:

* ``libfcmoe.so`` -- the HIP kernels and the C ABI of ``include/fcmoe.h``
  (``hipcc --offload-arch=gfx950``; no torch dependency);
* ``libfcmoe_probe.so`` -- the measurement probes ``bench.py --probe`` runs
  (``csrc/fcmoe_probe.h``); not part of the operator ABI;
* ``_moe_C<EXT_SUFFIX>`` -- the C++ torch extension that marshals tensors into
  that C ABI (g++ against the torch / ROCm headers, rpath ``$ORIGIN``).

Usage: ``python -m fused_cpp_amd.build`` (or ``build()``). hipcc cross-compiles
for gfx950 without a GPU. Compilation flags: ``-ffp-contract=off`` keeps each
binary32 operation separately rounded (the W8A8 path is bit-exact against the
CPU restatement of the reference arithmetic); packed-fp32 instructions are
disabled.
"""

from __future__ import annotations

import os
import re
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
ARCH = os.environ.get("FCMOE_OFFLOAD_ARCH", "gfx950")

HIP_SOURCES = ["fcmoe_api.hip", "fcmoe_route.hip", "fcmoe_quant.hip", "fcmoe_gemm.hip", "fcmoe_gemm_lds.hip", "fcmoe_gemm_smallm.hip", "fcmoe_combine.hip", "fcmoe_decode_tail.hip", "fcmoe_router.hip"]
# bench-only measurement probes: a library of their own (fcmoe_probe.h), linked against libfcmoe.so
PROBE_SOURCES = ["fcmoe_probe.hip"]
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++20",
    "-ffp-contract=off",
    # MFMA accumulators in ordinary VGPRs: avoids AGPR<->VGPR copy storms and
    # lets the 256-row tile run 2 waves/SIMD (234 VGPRs, no AGPRs)
    "-mllvm",
    "-amdgpu-mfma-vgpr-form=1",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]

LIB = PKG / "libfcmoe.so"
PROBE_LIB = PKG / "libfcmoe_probe.so"
EXT = PKG / ("_moe_C" + sysconfig.get_config_var("EXT_SUFFIX"))
BUILD_DIR = PKG / "_build"


def _run(cmd: list[str]) -> str:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout)
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd[:3])} ...")
    return proc.stdout


_SCRATCH_RE = re.compile(r"Function Name: (\S+).*?ScratchSize \[bytes/lane\]: (\d+)", re.S)


def _check_no_scratch(src: str, remarks: str) -> None:
    """Refuse kernels that spill to scratch: every kernel here is sized to keep
    its working set in registers, and a spill means a tile configuration
    exceeds the register budget it was designed for."""
    spilled = [(name, int(n)) for name, n in _SCRATCH_RE.findall(remarks) if int(n) > 0]
    if spilled:
        raise RuntimeError(f"{src}: kernels use scratch (register spills): {spilled[:4]}")


def build_lib(out_dir: Path | None = None, diag: int = 0) -> Path:
    """Compile every HIP source to an object in parallel, then link libfcmoe.so
    (and libfcmoe_probe.so). With out_dir, only libfcmoe.so is built, into
    out_dir, with the diagnostic bits `diag` of fcmoe_gemm_lds.hip (FCMOE_DIAG:
    timing-only variants and the persistent launches' item trace); the
    package's own library is always built without them."""
    lib_path = LIB if out_dir is None else Path(out_dir) / "libfcmoe.so"
    build_dir = BUILD_DIR if out_dir is None else Path(out_dir) / "_obj"
    build_dir.mkdir(parents=True, exist_ok=True)
    hipcc = str(ROCM / "bin" / "hipcc")
    flags = HIP_FLAGS + ([f"-DFCMOE_DIAG={int(diag)}"] if diag else [])

    def compile_one(src: str) -> str:
        obj = build_dir / (src + ".o")
        remarks = _run([hipcc, *flags, "-Rpass-analysis=kernel-resource-usage", "-c", str(CSRC / src), "-o",
                        str(obj)])
        _check_no_scratch(src, remarks)
        return str(obj)

    srcs = HIP_SOURCES + (PROBE_SOURCES if out_dir is None else [])
    with ThreadPoolExecutor(max_workers=min(len(srcs), os.cpu_count() or 1)) as ex:
        objs = dict(zip(srcs, ex.map(compile_one, srcs)))
    tmp = lib_path.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *[objs[s] for s in HIP_SOURCES]])
    os.replace(tmp, lib_path)
    if out_dir is not None:
        return lib_path
    tmp = PROBE_LIB.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *[objs[s] for s in PROBE_SOURCES],
          f"-L{PKG}", "-lfcmoe", "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, PROBE_LIB)
    return LIB


def build_ext() -> Path:
    """Compile the torch host extension against libfcmoe.so."""
    import torch
    from torch.utils import cpp_extension

    torch_lib = Path(torch.__file__).resolve().parent / "lib"
    incs = [*cpp_extension.include_paths(), sysconfig.get_paths()["include"], str(ROCM / "include")]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [
        os.environ.get("CXX", "g++"),
        "-O2",
        "-fPIC",
        "-shared",
        "-std=c++17",
        "-D__HIP_PLATFORM_AMD__=1",
        "-DUSE_ROCM=1",
        "-DTORCH_EXTENSION_NAME=_moe_C",
        "-DTORCH_API_INCLUDE_EXTENSION_H",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        *[f"-I{i}" for i in incs],
        str(CSRC / "moe_ext.cpp"),
        "-o",
        str(EXT) + ".tmp",
        f"-L{torch_lib}",
        f"-L{PKG}",
        "-lfcmoe",
        "-lc10",
        "-lc10_hip",
        "-ltorch",
        "-ltorch_cpu",
        "-ltorch_hip",
        "-ltorch_python",
        f"-L{ROCM / 'lib'}",
        "-lamdhip64",
        "-Wl,-rpath,$ORIGIN",
        f"-Wl,-rpath,{torch_lib}",
    ]
    _run(cmd)
    os.replace(str(EXT) + ".tmp", EXT)
    return EXT


def build() -> None:
    build_lib()
    build_ext()


if __name__ == "__main__":
    import argparse

    ap = argparse.ArgumentParser(description="build libfcmoe.so and the torch extension in-tree")
    ap.add_argument("--diag", type=int, default=0,
                    help="with --out: diagnostic bits of the LDS-staged GEMM (1 no epilogues, 2 no stage loads, "
                         "8 no fragment reads or MFMAs, 4 item trace); load the result with LD_LIBRARY_PATH=DIR FCMOE_LIB_DIR=DIR")
    ap.add_argument("--out", default=None, help="directory for a diagnostic libfcmoe.so (the package's is untouched)")
    args = ap.parse_args()
    if args.out:
        print(f"built {build_lib(Path(args.out), args.diag)}")
    else:
        if args.diag:
            raise SystemExit("--diag needs --out: the package's library is built without diagnostics")
        build()
        print(f"built {LIB.name} and {EXT.name}")
