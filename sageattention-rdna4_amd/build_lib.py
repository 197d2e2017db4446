"""Build libsagemi355.so, the gfx950 HIP library behind `sageattention`, in-tree.

    python sageattention-rdna4_amd/build_lib.py [--verbose]

Compiles every `csrc/*.hip` for `--offload-arch=gfx950` with hipcc (in parallel, one process per
translation unit) and links them into `sageattention/_lib/libsagemi355.so`. Flags that matter for
numerics: no fast-math (fp32 division stays correctly rounded), and packed-fp32 code generation
disabled (`-Xclang -target-feature -Xclang -packed-fp32-ops`).
"""
import concurrent.futures
import glob
import hashlib
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB_DIR = os.path.join(HERE, "sageattention", "_lib")
LIB_NAME = "libsagemi355.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
COMMON_FLAGS = [
    "--offload-arch=" + ARCH, "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-command-line-argument",
]


# Per-source extra flags. The main loop is built without NaN semantics: every max it takes is over
# finite scores or -inf masks, and with NaNs honoured each fmaxf would first quiet its inputs
# (one extra VALU instruction per operand on the softmax's critical path).
FILE_FLAGS = {
    "attn_fwd.hip": ["-fno-honor-nans"],
    "attn_fwd_pp.hip": ["-fno-honor-nans"],
    "attn_fwd_pl.hip": ["-fno-honor-nans"],
}


def lib_path():
    return os.path.join(LIB_DIR, LIB_NAME)


INCLUDE = os.path.join(os.path.dirname(HERE), "include")


def source_hash():
    """The build id: a SHA-256 prefix over every source the library is compiled from (csrc/*.hip,
    csrc/*.h, include/*.h, by name and content) and the compiler flags. The library returns the
    value it was built with from `sage_build_id()`, so a test can tell a stale library from one
    built from the tree it runs in."""
    h = hashlib.sha256()
    files = sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.h"))
                   + glob.glob(os.path.join(INCLUDE, "*.h")))
    for f in files:
        h.update(os.path.relpath(f, os.path.dirname(HERE)).encode())
        with open(f, "rb") as fh:
            h.update(fh.read())
    h.update(repr((COMMON_FLAGS, sorted(FILE_FLAGS.items()))).encode())
    return h.hexdigest()[:16]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature: harmless, not shown.
    noise = ("packed-fp32-ops", "is not a recognized feature for this target")
    err = "\n".join(l for l in res.stderr.splitlines() if not any(n in l for n in noise))
    if res.returncode != 0:
        raise RuntimeError("command failed (%d): %s\n%s" % (res.returncode, " ".join(cmd), err))
    if verbose and err.strip():
        print(err, file=sys.stderr)
    return res


def build(verbose=False, jobs=None):
    """Compile and link the library; returns its path. Always rebuilds."""
    os.makedirs(LIB_DIR, exist_ok=True)
    obj_dir = os.path.join(HERE, "_build")
    os.makedirs(obj_dir, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    if not sources:
        raise RuntimeError("no HIP sources under %s" % CSRC)
    objs = [os.path.join(obj_dir, os.path.splitext(os.path.basename(s))[0] + ".o") for s in sources]
    bid = ['-DSAGE_BUILD_ID="%s"' % source_hash()]
    cmds = [[HIPCC] + COMMON_FLAGS + FILE_FLAGS.get(os.path.basename(s), []) + bid
            + ["-c", s, "-o", o] for s, o in zip(sources, objs)]
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs or min(8, len(cmds))) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    out = lib_path()
    tmp = out + ".tmp"
    _run([HIPCC, "--offload-arch=" + ARCH, "-shared", "-fPIC", "-o", tmp] + objs, verbose)
    _check_kernel_stubs(tmp)
    os.replace(tmp, out)
    return out


def _check_kernel_stubs(lib):
    """Fail the build if a kernel's host launch stub is undefined. The host pass can drop a kernel
    template's stub without a diagnostic (a constraint check it cannot satisfy, deferred and never
    reported), and the library would then link and only fail to load."""
    nm = os.path.join(os.path.dirname(HIPCC), "..", "lib", "llvm", "bin", "llvm-nm")
    if not os.path.exists(nm):
        nm = "nm"
    res = subprocess.run([nm, "-u", lib], capture_output=True, text=True)
    missing = [l.split()[-1] for l in res.stdout.splitlines() if "__device_stub__" in l]
    if missing:
        raise RuntimeError("undefined kernel stubs in %s (a kernel was dropped by the host pass):\n%s"
                           % (lib, "\n".join(missing[:8])))


if __name__ == "__main__":
    print(build(verbose="--verbose" in sys.argv))
