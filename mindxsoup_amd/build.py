"""Ahead-of-time build of libmxs_nf4.so (the C-ABI library of the HIP kernels) for gfx950.

    python -m mindxsoup_amd.build        # or __graft_entry__.build()

Every csrc/*.hip file is compiled by hipcc to an object in csrc/_build/ (in parallel), then
linked into mindxsoup_amd/libmxs_nf4.so.  No torch headers are involved: the library's
interface is include/mxs_nf4.h.

csrc/probe/hbm_probe.hip (HBM rate probes bench.py reports; include/mxs_probe.h) is linked
apart into mindxsoup_amd/libmxs_probe.so, so the product library exports only the NF4 path.

csrc/torch_ops.cpp (host C++ only, no device code) is compiled by g++ against torch's headers
beside them and linked into mindxsoup_amd/libmxs_nf4_torch.so, which registers the
torch.ops.mxs_nf4 operators and links libmxs_nf4.so from its own directory.

Sources that issue global loads as inline asm (the ones calling vm_ready) are also compiled to
device assembly, which isa_check verifies: no instruction may name a register whose load can
still be in flight.  A finding fails the build.
"""

import concurrent.futures
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
OBJ = os.path.join(CSRC, "_build")
LIB = os.path.join(PKG, "libmxs_nf4.so")
TORCH_SRC = os.path.join(CSRC, "torch_ops.cpp")
TORCH_LIB = os.path.join(PKG, "libmxs_nf4_torch.so")
PROBE_SRC = os.path.join(CSRC, "probe", "hbm_probe.hip")
PROBE_LIB = os.path.join(PKG, "libmxs_probe.so")
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-fno-gpu-flush-denormals-to-zero",
    # no packed-fp32 instructions (v_pk_*_f32) in generated code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
    f"-I{os.path.join(ROOT, 'include')}", f"-I{CSRC}",
]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src):
    obj = os.path.join(OBJ, os.path.basename(src)[:-4] + ".o")
    cmd = [HIPCC, *FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so: harmless
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def _check_asm(src):
    """Compile `src` to gfx950 assembly and run the in-flight-register check on it."""
    from . import isa_check

    out = os.path.join(OBJ, os.path.basename(src)[:-4] + ".s")
    cmd = [HIPCC, *FLAGS, "--cuda-device-only", "-S", src, "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc -S failed on {src}:\n{r.stderr}")
    bad = isa_check.check(open(out).read())
    if bad:
        lines = []
        for name, rep in bad.items():
            lines.append(f"{name}: {len(rep)} uses of registers with a load in flight")
            lines += [f"   #{k}: {text}   pending {regs}" for k, text, regs in rep[:8]]
        raise RuntimeError(f"isa_check failed on {src} ({out}):\n" + "\n".join(lines))
    return out


def _torch_flags():
    import torch

    tp = os.path.dirname(os.path.abspath(torch.__file__))
    compile_flags = [
        "-O2", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
        f"-I{os.path.join(tp, 'include')}",
        f"-I{os.path.join(tp, 'include', 'torch', 'csrc', 'api', 'include')}",
        "-I/opt/rocm/include", f"-I{os.path.join(ROOT, 'include')}",
    ]
    link_flags = [f"-L{PKG}", "-lmxs_nf4", f"-L{os.path.join(tp, 'lib')}", "-lc10", "-lc10_hip",
                  "-ltorch_cpu", "-L/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath,$ORIGIN"]
    return compile_flags, link_flags


def _compile_torch_ops():
    obj = os.path.join(OBJ, "torch_ops.o")
    r = subprocess.run(["g++", *_torch_flags()[0], "-c", TORCH_SRC, "-o", obj],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"g++ failed on {TORCH_SRC}:\n{r.stderr}")
    return obj


def _link_torch_ops(obj):
    tmp = TORCH_LIB + ".tmp"
    r = subprocess.run(["g++", "-shared", obj, "-o", tmp, *_torch_flags()[1]],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link of {TORCH_LIB} failed:\n{r.stderr}")
    os.replace(tmp, TORCH_LIB)


def _link_hip(objs, lib):
    tmp = lib + ".tmp"
    r = subprocess.run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link of {lib} failed:\n{r.stderr}")
    os.replace(tmp, lib)


def build(verbose=True):
    os.makedirs(OBJ, exist_ok=True)
    srcs = sources()
    asm_srcs = [s for s in srcs if "vm_ready(" in open(s).read()]
    workers = min(len(srcs) + len(asm_srcs) + 2, max(1, (os.cpu_count() or 4)), 8)
    with concurrent.futures.ThreadPoolExecutor(workers) as ex:
        torch_obj = ex.submit(_compile_torch_ops)
        probe_obj = ex.submit(_compile, PROBE_SRC)
        checks = [ex.submit(_check_asm, s) for s in asm_srcs]
        objs = list(ex.map(_compile, srcs))
        for c in checks:
            c.result()
        torch_obj = torch_obj.result()
        probe_obj = probe_obj.result()
    _link_hip(objs, LIB)
    _link_hip([probe_obj], PROBE_LIB)
    _link_torch_ops(torch_obj)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources, {TORCH_LIB} and {PROBE_LIB}")
    return LIB


if __name__ == "__main__":
    build()
