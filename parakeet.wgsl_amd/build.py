"""Build the in-tree native libraries of the palette GEMM package.

    python parakeet.wgsl_amd/build.py            # everything
    python parakeet.wgsl_amd/build.py --lib      # libpk_palette.so only
    python parakeet.wgsl_amd/build.py --sanitize # the host-side ASan + UBSan variant

Outputs (git-ignored, shipped with the tree):
  lib/libpk_palette.so   HIP kernels for gfx950 + the C ABI (include/pk_palette.h)
  lib/pk_napi.node       Node N-API addon over the C ABI
  _san/libpk_palette.so, _san/pk_napi.node
                         the same with the host code (the C ABI translation
                         units and the addon) built with AddressSanitizer and
                         UndefinedBehaviorSanitizer against clang's shared
                         runtime; the device code is the regular build's. For
                         the CPU tests' sanitizer leg, never for the GPU.
"""
from __future__ import annotations

import argparse
import concurrent.futures
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
ADDON = os.path.join(PKG, "addon")
LIB = os.path.join(PKG, "lib")
OBJ = os.path.join(PKG, "_build")
INCLUDE = os.path.join(ROOT, "include")

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# Packed-f32 VALU ops are disabled for all device code (v_pk_*_f32).
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", INCLUDE, "-I", CSRC,
]
SOURCES = [
    "pk_abi.cpp", "pk_conv_abi.cpp", "pk_attention_abi.cpp", "pk_layernorm_abi.cpp",
    "pk_encoder_abi.cpp", "pk_subsampling_abi.cpp", "pk_tdt_abi.cpp", "pk_codes.hip", "pk_conv.hip",
    "pk_subsampling.hip", "pk_tdt.hip",
    "pk_attention.hip", "pk_layernorm.hip",
    "pk_gemm_f16.hip", "pk_gemm_f16k.hip",
    "pk_gemm_f16s.hip", "pk_gemm_f32.hip",
]
NODE_INCLUDE = "/usr/include/node"
SAN = os.path.join(PKG, "_san")
CLANG = "/opt/rocm/llvm/bin/clang"
# Host-only sanitizer flags (each after -Xarch_host on a hipcc line, so no
# device code is built with them).
SAN_HOST = ["-fsanitize=address", "-fsanitize=undefined", "-fno-sanitize-recover=undefined",
            "-fno-omit-frame-pointer", "-g"]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    noise = "is not a recognized feature for this target"
    out = "\n".join(line for line in proc.stdout.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out)


def _compile(source: str) -> str:
    src = os.path.join(CSRC, source)
    obj = os.path.join(OBJ, os.path.splitext(source)[0] + ".o")
    lang = ["-x", "hip"] if source.endswith(".cpp") else []
    _run([HIPCC, *HIP_FLAGS, *lang, "-c", src, "-o", obj])
    return obj


def build_lib(jobs: int | None = None) -> str:
    os.makedirs(OBJ, exist_ok=True)
    os.makedirs(LIB, exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 4, 16)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objects = list(pool.map(_compile, SOURCES))
    target = os.path.join(LIB, "libpk_palette.so")
    tmp = target + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objects,
          "-Wl,-soname,libpk_palette.so"])
    os.replace(tmp, target)
    return target


def sanitizer_runtime() -> str:
    """clang's shared AddressSanitizer runtime (it carries the UBSan handlers
    too): preload it into a process that loads a sanitized library."""
    import glob
    found = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not found:
        raise RuntimeError("clang's AddressSanitizer runtime is missing")
    return found[-1]


def _stale(target: str, sources: list[str]) -> bool:
    return not os.path.exists(target) or any(os.path.getmtime(s) > os.path.getmtime(target) for s in sources)


def build_sanitized(jobs: int | None = None) -> str:
    """_san/libpk_palette.so (the C ABI translation units with ASan + UBSan,
    linked with the regular build's kernel objects) and _san/pk_napi.node
    (the addon, likewise); rebuilt when a source is newer."""
    os.makedirs(SAN, exist_ok=True)
    abi_sources = [s for s in SOURCES if s.endswith(".cpp")]
    kernels = [os.path.join(OBJ, os.path.splitext(s)[0] + ".o") for s in SOURCES if s.endswith(".hip")]
    if any(not os.path.exists(k) for k in kernels):
        build_lib(jobs)
    headers = [os.path.join(d, f) for d in (CSRC, INCLUDE) for f in os.listdir(d) if f.endswith(".h")]
    flags = [f for flag in SAN_HOST for f in ("-Xarch_host", flag)]

    def compile_san(source: str) -> str:
        src = os.path.join(CSRC, source)
        obj = os.path.join(SAN, os.path.splitext(source)[0] + ".o")
        if _stale(obj, [src] + headers):
            _run([HIPCC, *HIP_FLAGS, *flags, "-x", "hip", "-c", src, "-o", obj])
        return obj
    jobs = jobs or min(len(abi_sources), os.cpu_count() or 4, 16)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objects = list(pool.map(compile_san, abi_sources))
    lib = os.path.join(SAN, "libpk_palette.so")
    if _stale(lib, objects + kernels):
        _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", lib + ".tmp", *objects, *kernels,
              "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined", "-shared-libasan",
              "-Wl,-soname,libpk_palette.so"])
        os.replace(lib + ".tmp", lib)
    source = os.path.join(ADDON, "pk_napi.c")
    addon = os.path.join(SAN, "pk_napi.node")
    if os.path.exists(os.path.join(NODE_INCLUDE, "node_api.h")) and _stale(addon, [source, lib] + headers):
        _run([CLANG, "-O1", "-g", "-std=gnu11", "-fPIC", "-shared", "-Wall", "-DNAPI_VERSION=8",
              "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined", "-fno-omit-frame-pointer",
              # globals uninstrumented: Node loads the addon so that its
              # string literals register twice (a false ODR report)
              "-mllvm", "-asan-globals=0",
              "-shared-libasan", "-I", NODE_INCLUDE, "-I", INCLUDE, source, "-o", addon + ".tmp",
              "-L", SAN, "-lpk_palette", "-Wl,-rpath,$ORIGIN"])
        os.replace(addon + ".tmp", addon)
    return lib


def build_addon() -> str | None:
    """Compile the N-API addon with gcc against the system Node headers."""
    source = os.path.join(ADDON, "pk_napi.c")
    if not os.path.exists(source):
        return None
    if not os.path.exists(os.path.join(NODE_INCLUDE, "node_api.h")):
        print("build: Node headers not found; skipping the N-API addon", file=sys.stderr)
        return None
    target = os.path.join(LIB, "pk_napi.node")
    tmp = target + ".tmp"
    cc = shutil.which("gcc") or "cc"
    _run([cc, "-O2", "-std=gnu11", "-fPIC", "-shared", "-Wall", "-Wextra", "-DNAPI_VERSION=8",
          "-I", NODE_INCLUDE, "-I", INCLUDE, source, "-o", tmp,
          "-L", LIB, "-lpk_palette", "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, target)
    return target


def main() -> None:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--lib", action="store_true", help="build only libpk_palette.so")
    parser.add_argument("--sanitize", action="store_true", help="build only the host-side sanitizer variant")
    args = parser.parse_args()
    if args.sanitize:
        print(build_sanitized())
        return
    print(build_lib())
    if not args.lib:
        addon = build_addon()
        if addon:
            print(addon)


if __name__ == "__main__":
    main()
