"""Ahead-of-time build of libmxs_nf4.so (the C-ABI library of the HIP kernels) for gfx950.

    python -m mindxsoup_amd.build        # or __graft_entry__.build()

Every csrc/*.hip file is compiled by hipcc to an object in csrc/_build/ (in parallel), then
linked into mindxsoup_amd/libmxs_nf4.so.  No torch headers are involved: the library's
interface is include/mxs_nf4.h.

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


def build(verbose=True):
    os.makedirs(OBJ, exist_ok=True)
    srcs = sources()
    asm_srcs = [s for s in srcs if "vm_ready(" in open(s).read()]
    workers = min(len(srcs) + len(asm_srcs), max(1, (os.cpu_count() or 4)), 8)
    with concurrent.futures.ThreadPoolExecutor(workers) as ex:
        checks = [ex.submit(_check_asm, s) for s in asm_srcs]
        objs = list(ex.map(_compile, srcs))
        for c in checks:
            c.result()
    tmp = LIB + ".tmp"
    r = subprocess.run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources")
    return LIB


if __name__ == "__main__":
    build()
