"""Build recipe for the MI355X libraries (run by __graft_entry__.build()).

  libpxk_gfx950.so      gfx950 HIP kernels behind the C ABI of include/pxk.h
  libpulsatrix_amd.so   C++17 host framework (DeviceBackend, MI355XBackend, modules, CausalLM)
                        and its C ABI, include/pulsatrix_amd.h

Both land in pulsatrix_amd/lib/ (in-tree, so they travel with the repository snapshot).
"""
import concurrent.futures
import glob
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB = os.path.join(HERE, "lib")
OBJ = os.path.join(HERE, "lib", "obj")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# -packed-fp32-ops: keep the compiler from emitting packed fp32 VALU ops.
DEVICE_FLAGS = ["--offload-arch=" + ARCH, "-std=c++17", "-O3", "-fPIC", "-Xclang", "-target-feature", "-Xclang",
                "-packed-fp32-ops", "-Wall", "-Wno-unused-result"]
HOST_FLAGS = ["-std=c++17", "-O2", "-fPIC", "-Wall"]
# Per-file additions. attention.hip: MFMA accumulators in VGPRs instead of AGPRs, so the online
# softmax's rescale of the context accumulators and the reads of each score tile need no
# v_accvgpr_read / v_accvgpr_write copies (36 per tile in the forward's key loop). Bitwise the same
# results; the statistics forward 15.4 -> 14.1 us at 1 x 512 tokens (9 / 3 heads of 64), 388 -> 364
# us at 8 x 1024 (32 / 8); the relevance kernels unchanged.
FILE_FLAGS = {"attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l and l.strip())
    if r.returncode != 0:
        raise RuntimeError("build failed: %s\n%s" % (" ".join(cmd), out))
    return out


def _compile(src, obj, flags, includes):
    if os.path.exists(obj) and os.path.getmtime(obj) >= max(
            [os.path.getmtime(src)] + [os.path.getmtime(h) for h in _headers(includes)]):
        return obj
    _run([HIPCC] + flags + ["-I" + i for i in includes] + ["-c", src, "-o", obj])
    return obj


def _headers(includes):
    out = []
    for d in includes:
        out += glob.glob(os.path.join(d, "**", "*.h"), recursive=True)
        out += glob.glob(os.path.join(d, "**", "*.hpp"), recursive=True)
    return out


def build_kernels(force=False):
    os.makedirs(OBJ, exist_ok=True)
    kdir = os.path.join(HERE, "csrc", "kernels")
    includes = [os.path.join(ROOT, "include"), kdir]
    srcs = sorted(glob.glob(os.path.join(kdir, "*.hip")))
    objs = [os.path.join(OBJ, "k_" + os.path.basename(s).replace(".hip", ".o")) for s in srcs]
    if force:
        for o in objs:
            if os.path.exists(o):
                os.remove(o)
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        list(ex.map(lambda so: _compile(so[0], so[1], DEVICE_FLAGS + FILE_FLAGS.get(os.path.basename(so[0]), []),
                                        includes), zip(srcs, objs)))
    out = os.path.join(LIB, "libpxk_gfx950.so")
    _run([HIPCC, "--offload-arch=" + ARCH, "-shared", "-fPIC", "-o", out] + objs)
    return out


def build_host(force=False):
    """The C++17 host framework, compiled by hipcc as host code and linked against libpxk."""
    hdir = os.path.join(HERE, "csrc", "host")
    srcs = sorted(glob.glob(os.path.join(hdir, "src", "*.cpp")))
    if not srcs:
        return None
    os.makedirs(OBJ, exist_ok=True)
    includes = [os.path.join(ROOT, "include"), os.path.join(hdir, "include")]
    flags = HOST_FLAGS + ["-D__HIP_PLATFORM_AMD__"]
    objs = [os.path.join(OBJ, "h_" + os.path.basename(s).replace(".cpp", ".o")) for s in srcs]
    if force:
        for o in objs:
            if os.path.exists(o):
                os.remove(o)
    with concurrent.futures.ThreadPoolExecutor(max_workers=8) as ex:
        list(ex.map(lambda so: _compile(so[0], so[1], flags, includes), zip(srcs, objs)))
    out = os.path.join(LIB, "libpulsatrix_amd.so")
    _run([HIPCC, "-shared", "-fPIC", "-o", out] + objs +
         ["-L" + LIB, "-lpxk_gfx950", "-Wl,-rpath,$ORIGIN", "-lpthread"])
    return out


def build_all(force=False):
    k = build_kernels(force)
    h = build_host(force)
    return k, h


if __name__ == "__main__":
    import sys

    print(build_all(force="--force" in sys.argv))
