"""Build recipe for libchonk.so (hipcc, gfx950) and the oracle's CPU library.

Run ``python -m chonklm_amd.build`` or call :func:`build_all`. Outputs stay
in-tree (``chonklm_amd/_lib/libchonk.so``, the Node addon
``chonklm_amd/_lib/chonk_napi.node``, ``oracle/_build/liborc.so``) so that
they travel with the repository snapshot to the GPU host.
"""
from __future__ import annotations

import os
import re
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
LIB_DIR = PKG / "_lib"
LIB_PATH = LIB_DIR / "libchonk.so"
OBJ_DIR = LIB_DIR / "obj"

HIP_SOURCES = [PKG / "csrc/hip/engine.hip", PKG / "csrc/hip/kernels.hip",
               PKG / "csrc/hip/prefill.hip", PKG / "csrc/hip/attn_decode.hip"]
HOST_SOURCES = [PKG / "csrc/host/gguf.cpp", PKG / "csrc/host/quantize.cpp", PKG / "csrc/host/synth.cpp"]
HEADERS = sorted((PKG / "csrc").rglob("*.h")) + [ROOT / "include/chonk.h"]

ARCH = os.environ.get("CHONK_OFFLOAD_ARCH", "gfx950")


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the ROCm toolchain is required to build libchonk.so")


def _run(cmd: list[str]) -> str:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass warns about the gfx-only target feature; keep other output
    lines = [ln for ln in proc.stdout.splitlines() if "packed-fp32-ops' is not a recognized" not in ln]
    if proc.returncode != 0:
        raise RuntimeError("build step failed: " + " ".join(cmd) + "\n" + "\n".join(lines))
    return proc.stdout


def _attn_dec_admitted(group: int, hd: int, walk: bool) -> bool:
    """The engine's rule for the register-resident decode attention (attn_dec_supported)."""
    return group * hd <= 1536 and not (hd == 256 and group >= 6 and walk)


def check_attn_dec_scratch(remarks: str) -> None:
    """Every k_attn_dec instance the engine may pick keeps its registers (no scratch):
    the kernel-resource-usage remarks of attn_decode.hip are read back here."""
    name = None
    bad = []
    for line in remarks.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            name = m.group(1)
            continue
        m = re.search(r"ScratchSize \[bytes/lane\]: (\d+)", line)
        g = re.search(r"k_attn_decILi(\d+)ELi(\d+)ELb(\d)", name or "")
        if m and g and int(m.group(1)) > 0:
            group, hd, walk = int(g.group(1)), int(g.group(2)), g.group(3) == "1"
            if _attn_dec_admitted(group, hd, walk):
                bad.append(f"k_attn_dec<{group}, {hd}, {str(walk).lower()}> ({m.group(1)} bytes per lane)")
    if bad:
        raise RuntimeError("decode attention instances the engine may pick spill to scratch: " + ", ".join(bad))


def build_library(jobs: int = 8) -> Path:
    """Compiles every source (always) and links libchonk.so."""
    hipcc = _hipcc()
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    common = ["-O3", "-std=c++20", "-fPIC", f"-I{ROOT / 'include'}", "-Wall", "-Wno-unused-function"]
    gpu = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
    jobs_list = []
    for src in HIP_SOURCES:
        obj = OBJ_DIR / (src.stem + ".o")
        extra = ["-Rpass-analysis=kernel-resource-usage"] if src.name == "attn_decode.hip" else []
        jobs_list.append((obj, [hipcc, *gpu, *common, *extra, "-c", str(src), "-o", str(obj)]))
    for src in HOST_SOURCES:
        obj = OBJ_DIR / (src.stem + ".host.o")
        jobs_list.append((obj, ["g++", "-O2", "-std=c++17", "-fPIC", "-Wall", "-c", str(src), "-o", str(obj)]))
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        outs = list(ex.map(lambda j: _run(j[1]), jobs_list))
    for (obj, _), out in zip(jobs_list, outs):
        if obj.stem == "attn_decode":
            check_attn_dec_scratch(out)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([hipcc, *gpu, "-shared", "-fPIC", "-o", str(tmp), *[str(o) for o, _ in jobs_list], "-lpthread"])
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


NAPI_SOURCE = PKG / "csrc/napi/chonk_napi.cpp"
NAPI_PATH = LIB_DIR / "chonk_napi.node"


def _node_include() -> Path | None:
    for cand in (Path("/usr/include/node"), Path("/usr/local/include/node")):
        if (cand / "node_api.h").exists():
            return cand
    return None


def build_napi() -> Path | None:
    """Builds the Node N-API addon over libchonk.so (skipped when Node's headers are absent)."""
    inc = _node_include()
    if inc is None:
        return None
    tmp = NAPI_PATH.with_suffix(".node.tmp")
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-DNODE_GYP_MODULE_NAME=chonk_napi",
          f"-I{inc}", f"-I{ROOT / 'include'}", str(NAPI_SOURCE), "-o", str(tmp), f"-L{LIB_DIR}", "-lchonk",
          "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, NAPI_PATH)
    return NAPI_PATH


def build_oracle() -> Path | None:
    """Builds the oracle's CPU restatement (test infrastructure)."""
    oracle = ROOT / "oracle"
    if not (oracle / "Makefile").exists():
        return None
    _run(["make", "-s", "-B", "-C", str(oracle)])
    return oracle / "_build" / "liborc.so"


def build_all(jobs: int = 8) -> None:
    build_library(jobs)
    build_napi()
    build_oracle()


if __name__ == "__main__":
    build_all(int(sys.argv[1]) if len(sys.argv) > 1 else 8)
    print(LIB_PATH)
