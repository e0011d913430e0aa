"""Builds the native libraries of this package, in-tree, for gfx950.

  libgn_bwd.so          HIP kernels + the C ABI declared in include/gn_bwd.h
  libgn_probe.so        measurement kernels of include/gn_probe.h (bench.py --ceilings only)
  _grilly_core*.so      pybind11 module, imported through grilly_core.py: tape engine (TensorRef,
                        OpType, Node, TapeArena,
                        BackwardEngine, TapeContext) calling libgn_bwd through the C ABI

Usage: python grilly-next_amd/build_native.py   (also called by __graft_entry__.build()).
Compiles every time it is called; objects go to grilly-next_amd/_build/.
"""
import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
INCLUDE = os.path.join(ROOT, "include")
ARCH = os.environ.get("GN_OFFLOAD_ARCH", "gfx950")

KERNEL_SOURCES = ["gn_errors.cpp", "gn_elementwise.hip", "gn_norm.hip", "gn_gemm.hip", "gn_gemm_dma.hip",
                  "gn_gemm_dma_f32a.hip", "gn_gemm_dma_f32b.hip", "gn_gemm_dma_bf16.hip",
                  "gn_gemm_dma_glu.hip", "gn_vsa.hip", "gn_attn.hip", "gn_optim.hip", "gn_tapeops.hip",
                  "gn_fwd.hip", "gn_skinny.hip", "gn_vsa_fwd.hip", "gn_gemm_f32.hip", "gn_lane.cpp"]
# measurement kernels for bench.py --ceilings, kept out of the backward library
PROBE_SOURCES = ["gn_probe.hip"]
TAPE_SOURCES = ["tape/autograd.cpp", "tape/device.cpp", "tape/checkpoint.cpp", "tape/hypernet.cpp",
                "tape/op_graph.cpp", "bindings.cpp"]

# -packed-fp32-ops off: packed fp32 VALU forms are kept out of the generated code.
HIP_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-I", INCLUDE, "-I", CSRC,
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wall",
             "-Wno-unused-function", "-Wno-unused-variable"]


# Extra flags per source.  gn_attn.hip: MFMAs in their VGPR form — the attention kernels
# keep P and dS in VGPRs between MFMAs, and the AGPR form made the register allocator
# shuttle every accumulator between the two files on each loop iteration.
FILE_FLAGS = {"gn_attn.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}


def _run(cmd):
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in p.stdout.splitlines() if "packed-fp32-ops" not in l)
    if p.returncode != 0:
        raise RuntimeError("build failed: " + " ".join(cmd) + "\n" + out)
    return out


def _obj(src):
    return os.path.join(BUILD, src.replace("/", "_").rsplit(".", 1)[0] + ".o")


def build_kernels(jobs=8):
    os.makedirs(BUILD, exist_ok=True)
    srcs = KERNEL_SOURCES + PROBE_SOURCES
    # the longest compiles first, so the pool's tail is short
    srcs.sort(key=lambda s: -os.path.getsize(os.path.join(CSRC, s)))
    cmds = [["hipcc", *HIP_FLAGS, *FILE_FLAGS.get(s, []), "-c", os.path.join(CSRC, s), "-o", _obj(s)]
            for s in srcs]
    with ThreadPoolExecutor(jobs) as ex:
        list(ex.map(_run, cmds))
    link_kernels()
    return os.path.join(HERE, "libgn_bwd.so")


def link_kernels():
    """libgn_bwd.so (the C ABI of include/gn_bwd.h) and libgn_probe.so (include/gn_probe.h)."""
    for name, srcs in (("libgn_bwd.so", KERNEL_SOURCES),
                       ("libgn_probe.so", PROBE_SOURCES + ["gn_errors.cpp"])):
        out = os.path.join(HERE, name)
        _run(["hipcc", "-shared", f"--offload-arch={ARCH}", "-o", out + ".tmp",
              *[_obj(s) for s in srcs]])
        os.replace(out + ".tmp", out)


def build_tape(jobs=8, extra=()):
    """extra: flags added to every compile and to the link (e.g. sanitizers)."""
    import pybind11
    os.makedirs(BUILD, exist_ok=True)
    py_inc = sysconfig.get_paths()["include"]
    ext = sysconfig.get_config_var("EXT_SUFFIX")
    flags = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-I", INCLUDE, "-I", CSRC,
             "-I", os.path.join(CSRC, "tape"), "-I", pybind11.get_include(), "-I", py_inc,
             "-D__HIP_PLATFORM_AMD__", "-I", "/opt/rocm/include", "-fvisibility=hidden", *extra]
    cmds = [["g++", *flags, "-c", os.path.join(CSRC, s), "-o", _obj(s)] for s in TAPE_SOURCES]
    with ThreadPoolExecutor(jobs) as ex:
        list(ex.map(_run, cmds))
    # the extension is _grilly_core; grilly_core.py loads it after torch (see there).  A
    # grilly_core*.so left by an older build would shadow grilly_core.py: remove it.
    for f in os.listdir(HERE):
        if f.startswith("grilly_core.") and f.endswith(".so"):
            os.remove(os.path.join(HERE, f))
    out = os.path.join(HERE, "_grilly_core" + ext)
    _run(["g++", "-shared", *extra, "-o", out + ".tmp", *[_obj(s) for s in TAPE_SOURCES],
          "-L", HERE, "-lgn_bwd", "-Wl,-rpath,$ORIGIN", "-L/opt/rocm/lib", "-lamdhip64",
          "-Wl,-rpath,/opt/rocm/lib"])
    os.replace(out + ".tmp", out)
    return out


def main():
    print(build_kernels())
    if all(os.path.exists(os.path.join(CSRC, s)) for s in TAPE_SOURCES):
        print(build_tape())


if __name__ == "__main__":
    sys.exit(main())
