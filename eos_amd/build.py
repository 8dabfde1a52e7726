"""Build recipe for the eoship library (gfx950 only).

1. Each device source under ``csrc/kernels`` is compiled offline into a gfx950
   code object with ``hipcc --genco`` (no run-time compiler, the counterpart of
   the reference's NVRTC step in runtime/backends/cuda/native_linux.go:500-588).
2. The code objects are linked into the shared library as read-only data
   (``.incbin``) and loaded at runtime creation with ``hipModuleLoadData``.
3. The host shim (plain C++ over the HIP runtime API) is compiled with g++ into
   ``eos_amd/libeoship.so``, together with the objects hipcc builds from the
   host sources that declare device variables (the static scratch of the
   no-allocation entry points).
4. A measurement code object (``_build/probe.hsaco``: MFMA rate and shader
   clock against operand data) is built for bench.py and not linked in.

Run ``python -m eos_amd.build`` or call :func:`build`.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
LIB_PATH = os.path.join(PKG_DIR, "libeoship.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = "gfx950"

# (code object symbol stem, device source)
DEVICE_SOURCES = [
    ("tq", os.path.join(CSRC, "kernels", "tq_kernels.hip")),
    ("enc", os.path.join(CSRC, "kernels", "enc_kernels.hip")),
    ("ret", os.path.join(CSRC, "kernels", "ret_kernels.hip")),
]
# Extra flags per code object. The encoder kernels are built without the
# mixed-precision FMA instructions (v_fma_mix*): the compiler folds some
# `(half)fmaf(a, b, c)` into one of them, which rounds the exact result to
# f16 once, and leaves others as an f32 FMA and a conversion, which round
# twice; which epilogue element gets which form depends on its position in
# the unrolled tile, so a row's values would depend on where the row lies in
# the batch. Without them every element is an f32 FMA rounded to f32, then
# to f16.
DEVICE_FLAGS = {
    "enc": ["-Xclang", "-target-feature", "-Xclang", "-fma-mix-insts"],
}
# Measurement code object for bench.py (MFMA rate and shader clock against
# operand data), built beside the library and not linked into it.
PROBE_SOURCE = os.path.join(CSRC, "kernels", "probe_kernels.hip")
PROBE_PATH = os.path.join(BUILD_DIR, "probe.hsaco")
# Host translation units that hold device variables (hipcc, host + device).
HIP_HOST_SOURCES = [
    os.path.join(CSRC, "eoship_noalloc.hip"),
]
HOST_SOURCES = [
    os.path.join(CSRC, "eoship_runtime.cpp"),
    os.path.join(CSRC, "eoship_tq.cpp"),
    os.path.join(CSRC, "eoship_encoder.cpp"),
    os.path.join(CSRC, "eoship_embed.cpp"),
    os.path.join(CSRC, "eoship_mll.cpp"),
    os.path.join(CSRC, "eoship_retrieval.cpp"),
]

# Packed-FP32 instructions are disabled for every device build.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print("+", " ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(
            f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")


def build(verbose: bool = False) -> str:
    """Compile every gfx950 code object and the host shim; return the .so path."""
    hipcc = shutil.which("hipcc") or os.path.join(ROCM, "bin", "hipcc")
    os.makedirs(BUILD_DIR, exist_ok=True)
    blobs = []
    for stem, src in DEVICE_SOURCES:
        out = os.path.join(BUILD_DIR, f"{stem}.hsaco")
        _run([hipcc, *HIPCC_FLAGS, *DEVICE_FLAGS.get(stem, []), "--genco", "-I",
              os.path.join(CSRC, "kernels"), "-o", out, src], verbose)
        blobs.append((stem, out))
    _run([hipcc, *HIPCC_FLAGS, "--genco", "-o", PROBE_PATH, PROBE_SOURCE], verbose)
    asm = [".section .note.GNU-stack,\"\",@progbits"]
    for stem, path in blobs:
        asm += [
            f".section .rodata.eoship_{stem},\"a\",@progbits",
            ".balign 4096",
            f".globl eoship_{stem}_co_begin",
            f"eoship_{stem}_co_begin:",
            f".incbin \"{path}\"",
            f".globl eoship_{stem}_co_end",
            f"eoship_{stem}_co_end:",
            ".byte 0",
        ]
    hip_objs = []
    for src in HIP_HOST_SOURCES:
        obj = os.path.join(BUILD_DIR, os.path.splitext(os.path.basename(src))[0] + ".o")
        _run([hipcc, *HIPCC_FLAGS, "-fPIC", "-c", "-I", os.path.join(REPO_DIR, "include"), "-I", CSRC,
              "-o", obj, src], verbose)
        hip_objs.append(obj)
    asm_path = os.path.join(BUILD_DIR, "eoship_blobs.S")
    with open(asm_path, "w") as f:
        f.write("\n".join(asm) + "\n")
    tmp = LIB_PATH + ".tmp"
    _run([
        "g++", "-O2", "-g", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wextra",
        "-Wno-unused-parameter", "-Wno-unused-result", "-D__HIP_PLATFORM_AMD__",
        "-I", os.path.join(REPO_DIR, "include"), "-I", CSRC, "-I", os.path.join(ROCM, "include"),
        *HOST_SOURCES, *hip_objs, asm_path,
        "-L", os.path.join(ROCM, "lib"), "-lamdhip64", f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}",
        "-Wl,--no-undefined", "-o", tmp,
    ], verbose)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


ASAN_LIB_PATH = os.path.join(BUILD_DIR, "libeoship_asan.so")


def build_sanitized(verbose: bool = False) -> str:
    """The host shim built with AddressSanitizer and UndefinedBehaviorSanitizer
    (host code only; the gfx950 code objects and the device-variable objects
    of build() are linked in unchanged) into _build/libeoship_asan.so. For
    CPU tests of the host-side parsers and argument checks, loaded by a
    process that preloads the sanitizer runtimes."""
    asm_path = os.path.join(BUILD_DIR, "eoship_blobs.S")
    hip_objs = [os.path.join(BUILD_DIR, os.path.splitext(os.path.basename(src))[0] + ".o")
                for src in HIP_HOST_SOURCES]
    if not os.path.exists(asm_path) or not all(os.path.exists(o) for o in hip_objs):
        build(verbose)
    tmp = ASAN_LIB_PATH + ".tmp"
    _run([
        "g++", "-O1", "-g", "-std=c++17", "-fPIC", "-shared", "-fno-omit-frame-pointer",
        "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined",
        "-Wno-unused-result", "-D__HIP_PLATFORM_AMD__",
        "-I", os.path.join(REPO_DIR, "include"), "-I", CSRC, "-I", os.path.join(ROCM, "include"),
        *HOST_SOURCES, *hip_objs, asm_path,
        "-L", os.path.join(ROCM, "lib"), "-lamdhip64", f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}",
        "-o", tmp,
    ], verbose)
    os.replace(tmp, ASAN_LIB_PATH)
    return ASAN_LIB_PATH


if __name__ == "__main__":
    if "--sanitize" in sys.argv:
        print(build_sanitized(verbose="-v" in sys.argv))
    else:
        print(build(verbose="-v" in sys.argv))
