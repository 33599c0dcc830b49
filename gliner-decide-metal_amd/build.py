"""Builds libgliner_decide_hip.so for gfx950 with hipcc.

Every source under csrc/ is compiled as HIP (device code for gfx950 only,
packed-fp32 instructions disabled) into objects under _build/, then linked
into lib/libgliner_decide_hip.so.  The decision front end under
csrc/frontend/ is host C++ and is built with g++ (linked against ICU) into
lib/libgliner_decide_frontend.so.  Run `python build.py` or call `build()`
(both libraries).
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_DIR = PKG_DIR / "lib"
LIB_PATH = LIB_DIR / "libgliner_decide_hip.so"
ARCH = "gfx950"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    "-Wno-unused-command-line-argument",
    # No packed fp32 VALU forms (v_pk_add/mul/fma_f32) in the generated code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{REPO / 'include'}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build the library)")


def _compile(src: Path, obj: Path) -> tuple[Path, int, str]:
    cmd = [hipcc(), "-x", "hip", "-c", str(src), "-o", str(obj), *COMMON_FLAGS]
    p = subprocess.run(cmd, capture_output=True, text=True)
    log = p.stdout + p.stderr
    # hipcc's host pass does not know the packed-fp32 feature; drop that note.
    log = "\n".join(line for line in log.splitlines() if "packed-fp32-ops" not in line)
    return src, p.returncode, log


FRONTEND_SRC = CSRC / "frontend"
FRONTEND_LIB_PATH = LIB_DIR / "libgliner_decide_frontend.so"
# The decision front end is host code: g++ against ICU (regex, grapheme
# clusters, case mapping, normal forms).
FRONTEND_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-fvisibility=hidden", "-Wall", "-Wextra",
                  f"-I{REPO / 'include'}", f"-I{FRONTEND_SRC}"]
FRONTEND_LIBS = ["-licui18n", "-licuuc", "-licudata"]


def build_frontend(verbose: bool = False) -> Path:
    """Builds libgliner_decide_frontend.so (CPU only) with g++."""
    BUILD_DIR.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    cxx = os.environ.get("CXX") or shutil.which("g++") or "g++"
    sources = sorted(FRONTEND_SRC.glob("*.cpp"))
    objs = [BUILD_DIR / ("frontend_" + s.name + ".o") for s in sources]

    def one(pair):
        src, obj = pair
        p = subprocess.run([cxx, "-c", str(src), "-o", str(obj), *FRONTEND_FLAGS], capture_output=True, text=True)
        return src, p.returncode, p.stdout + p.stderr

    with cf.ThreadPoolExecutor(max_workers=max(1, min(len(sources), 4))) as ex:
        results = list(ex.map(one, zip(sources, objs)))
    failures = [f"--- {src.name} ---\n{log}" for src, rc, log in results if rc != 0]
    if failures:
        raise RuntimeError("front-end compilation failed:\n" + "\n".join(failures))
    if verbose:
        for src, _, log in results:
            if log.strip():
                print(f"--- {src.name} ---\n{log}", file=sys.stderr)
    tmp = FRONTEND_LIB_PATH.with_suffix(".so.tmp")
    p = subprocess.run([cxx, "-shared", "-o", str(tmp), *map(str, objs), *FRONTEND_LIBS], capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError("front-end link failed:\n" + p.stdout + p.stderr)
    os.replace(tmp, FRONTEND_LIB_PATH)
    return FRONTEND_LIB_PATH


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    BUILD_DIR.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    sources = sorted([*CSRC.glob("*.hip"), *CSRC.glob("*.cpp")])
    if not sources:
        raise RuntimeError(f"no sources under {CSRC}")
    objs = [BUILD_DIR / (s.name + ".o") for s in sources]
    jobs = jobs or min(len(sources), max(1, min(os.cpu_count() or 1, 8)))
    failures = []
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for src, rc, log in ex.map(lambda a: _compile(*a), zip(sources, objs)):
            if rc != 0:
                failures.append(f"--- {src.name} ---\n{log}")
            elif verbose and log.strip():
                print(f"--- {src.name} ---\n{log}", file=sys.stderr)
    if failures:
        raise RuntimeError("HIP compilation failed:\n" + "\n".join(failures))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), "-shared", f"--offload-arch={ARCH}", "-fPIC", "-o", str(tmp), *map(str, objs)]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError("link failed:\n" + p.stdout + p.stderr)
    os.replace(tmp, LIB_PATH)
    build_frontend(verbose)
    build_sanitized(verbose)
    return LIB_PATH


# ---------------------------------------------------------------------------
# Host sanitizer build: the host C++ that parses untrusted input (the
# safetensors reader and the C-ABI around it; the tokenizer.json / charsmap /
# schema front end) with AddressSanitizer and UndefinedBehaviorSanitizer, into
# lib/sanitize/.  Device code is built exactly as in build(): each sanitizer
# flag on a hipcc line is host-only (-Xarch_host).  tests/test_sanitized_host.py
# runs the CPU tests of these paths against this build.
# ---------------------------------------------------------------------------
SAN_DIR = LIB_DIR / "sanitize"
SAN_HOST_SOURCES = ("weights.cpp", "capi.cpp", "model.cpp")
SAN_HOST_FLAGS = [
    "-Xarch_host", "-fsanitize=address",
    "-Xarch_host", "-fsanitize=undefined",
    "-Xarch_host", "-fno-omit-frame-pointer",
]
SAN_CXX_FLAGS = [
    "-fsanitize=address,undefined",
    "-fno-omit-frame-pointer",
    "-shared-libsan",
]


def llvm_dir() -> Path:
    return Path(hipcc()).resolve().parent.parent / "lib" / "llvm"


def asan_runtime() -> Path:
    """The clang AddressSanitizer runtime both sanitized libraries link (to
    LD_PRELOAD into an unsanitized interpreter)."""
    found = sorted(llvm_dir().glob("lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not found:
        raise RuntimeError("clang AddressSanitizer runtime not found")
    return found[-1]


def build_sanitized(verbose: bool = False) -> tuple[Path, Path]:
    BUILD_DIR.mkdir(exist_ok=True)
    SAN_DIR.mkdir(parents=True, exist_ok=True)

    def run(cmd):
        p = subprocess.run(cmd, capture_output=True, text=True)
        log = "\n".join(line for line in (p.stdout + p.stderr).splitlines() if "packed-fp32-ops" not in line)
        return p.returncode, log

    # HIP library: the sanitized host objects linked with the regular device objects.
    def one_hip(name):
        obj = BUILD_DIR / f"san_{name}.o"
        rc, log = run([hipcc(), "-x", "hip", "-c", str(CSRC / name), "-o", str(obj), *COMMON_FLAGS, "-g",
                       *SAN_HOST_FLAGS])
        return name, obj, rc, log

    clangxx = str(llvm_dir() / "bin" / "clang++")

    def one_fe(src):
        obj = BUILD_DIR / f"san_frontend_{src.name}.o"
        rc, log = run([clangxx, "-c", str(src), "-o", str(obj), *FRONTEND_FLAGS, "-g", *SAN_CXX_FLAGS])
        return src.name, obj, rc, log

    fe_sources = sorted(FRONTEND_SRC.glob("*.cpp"))
    with cf.ThreadPoolExecutor(max_workers=6) as ex:
        hip_res = list(ex.map(one_hip, SAN_HOST_SOURCES))
        fe_res = list(ex.map(one_fe, fe_sources))
    failures = [f"--- {n} ---\n{log}" for n, _, rc, log in hip_res + fe_res if rc != 0]
    if failures:
        raise RuntimeError("sanitized compilation failed:\n" + "\n".join(failures))
    regular = [BUILD_DIR / (s.name + ".o") for s in sorted(CSRC.glob("*.hip"))]
    hip_lib = SAN_DIR / LIB_PATH.name
    rc, log = run([hipcc(), "-shared", f"--offload-arch={ARCH}", "-fPIC", "-o", str(hip_lib),
                   *[str(o) for _, o, _, _ in hip_res], *map(str, regular), "-shared-libsan", *SAN_HOST_FLAGS[:4]])
    if rc != 0:
        raise RuntimeError("sanitized link failed:\n" + log)
    fe_lib = SAN_DIR / FRONTEND_LIB_PATH.name
    rc, log = run([clangxx, "-shared", "-o", str(fe_lib), *[str(o) for _, o, _, _ in fe_res], *SAN_CXX_FLAGS,
                   *FRONTEND_LIBS])
    if rc != 0:
        raise RuntimeError("sanitized front-end link failed:\n" + log)
    return hip_lib, fe_lib


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
    print(FRONTEND_LIB_PATH)
