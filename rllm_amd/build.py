"""Ahead-of-time build of librq.so for gfx950.

1. hipcc --genco compiles each kernel source (csrc/rq_kernels.hip: the Q8_1
   pass and the dot4 matvecs; csrc/rq_mmq.hip: the int8-MFMA matvecs) into
   one gfx950 code object each.
2. An assembler stub (.incbin) embeds the code objects in the library.
3. hipcc compiles csrc/rq_static.hip (the fixed device scratch of
   rq_matmul_many_noalloc) as an ordinary host + device object.
4. g++ compiles the host side (csrc/rq_host.cpp) against the HIP runtime and
   links everything into the library.

The result, rllm_amd/lib/librq.so, is self-contained: rq_open() loads the
embedded code objects with hipModuleLoadData; nothing is compiled at run time.
The same steps with -DRQ_TIMELINE build rllm_amd/lib/librq_tl.so, whose
kernels also record per-wave timestamps (include/rq_timeline.h; only
bench.py --timeline loads it).

Usage: python -m rllm_amd.build   (or rllm_amd.build.build()).
"""
from __future__ import annotations

import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIBDIR = os.path.join(PKG, "lib")
LIB = os.path.join(LIBDIR, "librq.so")
# bench.py's roofline reference (a read-only kernel of the matvec's launch
# shape); not part of librq.so.
FLOOR_LIB = os.path.join(LIBDIR, "librq_floor.so")
# librq.so with per-wave timestamps (bench.py --timeline).
TIMELINE_LIB = os.path.join(LIBDIR, "librq_tl.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = "gfx950"
# Kernel sources, one code object each (embedded as <name>_blob).
KERNEL_SOURCES = ("rq_kernels", "rq_mmq")

# Device code: IEEE-correct f32 division (the Q8_1 scale and codes must match
# the CPU bit for bit) and no packed-f32 instructions (they have given wrong
# results on these machines).
HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]


def _check(cmd: list[str], returncode: int, output: str) -> None:
    out = "\n".join(l for l in output.splitlines() if "packed-fp32-ops" not in l)
    if returncode != 0:
        raise RuntimeError(f"build step failed ({returncode}): {' '.join(cmd)}\n{out}")


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    _check(cmd, r.returncode, r.stdout)


def _run_all(cmds: list[list[str]]) -> None:
    """Runs independent compile steps at once; fails on the first failure."""
    procs = [(c, subprocess.Popen(c, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)) for c in cmds]
    results = [(c, p.communicate()[0], p.returncode) for c, p in procs]
    for c, out, rc in results:
        _check(c, rc, out)


def _blob_stub(builddir: str, tag: str) -> str:
    """The assembler stub embedding the code objects <name><tag>.hsaco."""
    stub = []
    for name in KERNEL_SOURCES:
        hsaco = os.path.join(builddir, f"{name}{tag}.hsaco")
        stub += [
            "    .section .rodata\n",
            "    .balign 4096\n",
            f"    .globl {name}_blob\n",
            f"    .type {name}_blob, @object\n",
            f"{name}_blob:\n",
            f'    .incbin "{hsaco}"\n',
            "    .byte 0\n",
            f"    .size {name}_blob, . - {name}_blob\n",
        ]
    stub.append('    .section .note.GNU-stack,"",@progbits\n')
    blob = os.path.join(builddir, f"rq_blob{tag}.S")
    with open(blob, "w") as f:
        f.write("".join(stub))
    return blob


def _link(csrc: str, blob: str, static_obj: str, out: str, defines: list[str]) -> list[str]:
    return [
        "g++", "-shared", "-fPIC", "-O2", "-std=c++17", "-Wall", "-Wextra", *defines,
        "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include", f"-I{csrc}",
        os.path.join(csrc, "rq_host.cpp"), os.path.join(csrc, "rq_gguf.cpp"), blob, static_obj,
        f"-L{ROCM}/lib", "-lamdhip64", "-lrocblas", f"-Wl,-rpath,{ROCM}/lib",
        "-o", out,
    ]


def build(verbose: bool = False, csrc: str = CSRC, libdir: str = LIBDIR, builddir: str = BUILD,
          floor: bool = True, timeline: bool = True) -> str:
    """Compile everything; returns the library path. `csrc`, `libdir` and
    `builddir` default to the package's own (a build of another source tree
    goes elsewhere); the kernel sources compile in parallel."""
    os.makedirs(builddir, exist_ok=True)
    os.makedirs(libdir, exist_ok=True)
    hipcc = os.path.join(ROCM, "bin", "hipcc")
    lib = os.path.join(libdir, "librq.so")
    static_obj = os.path.join(builddir, "rq_static.o")
    tags = ["", "_tl"] if timeline else [""]
    jobs = [[hipcc, "--genco", *HIPCC_FLAGS, *(["-DRQ_TIMELINE"] if tag else []), f"-I{csrc}",
             os.path.join(csrc, f"{name}.hip"), "-o", os.path.join(builddir, f"{name}{tag}.hsaco")]
            for tag in tags for name in KERNEL_SOURCES]
    # The fixed scratch of rq_matmul_many_noalloc: a device array in a HIP
    # translation unit of its own (host + gfx950 device code, registered with
    # the HIP runtime when the library loads).
    jobs.append([hipcc, "-c", "-fPIC", *HIPCC_FLAGS, f"-I{csrc}", os.path.join(csrc, "rq_static.hip"), "-o", static_obj])
    floor_lib = os.path.join(libdir, "librq_floor.so")
    if floor:
        # bench.py's read-floor probe (rq_floor.hip), a library of its own.
        jobs.append([hipcc, "-shared", "-fPIC", *HIPCC_FLAGS, f"-I{csrc}", os.path.join(csrc, "rq_floor.hip"), "-o",
                     floor_lib + ".tmp"])
    _run_all(jobs)
    tmp = lib + ".tmp"
    links = [_link(csrc, _blob_stub(builddir, ""), static_obj, tmp, [])]
    tl_lib = os.path.join(libdir, "librq_tl.so")
    if timeline:
        links.append(_link(csrc, _blob_stub(builddir, "_tl"), static_obj, tl_lib + ".tmp", ["-DRQ_TIMELINE"]))
    _run_all(links)
    os.replace(tmp, lib)
    if timeline:
        os.replace(tl_lib + ".tmp", tl_lib)
    if floor:
        os.replace(floor_lib + ".tmp", floor_lib)
    if verbose:
        print(f"built {lib}" + (f" and {floor_lib}" if floor else ""))
    return lib


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
