"""Builds libsuf_hip.so (gfx950) in-tree with hipcc.

    python -m suf_amd.build          # from the repository root

Each .hip translation unit under suf_amd/csrc is compiled to an object file
under suf_amd/lib/obj and linked into suf_amd/lib/libsuf_hip.so.  The build
always recompiles (it is the "does it build" check); pass --if-stale to skip
units whose object file is newer than every source and header.
"""
import argparse
import glob
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIBDIR = os.path.join(PKG, "lib")
OBJDIR = os.path.join(LIBDIR, "obj")
LIB = os.path.join(LIBDIR, "libsuf_hip.so")
ARCH = "gfx950"

HIPCC_FLAGS = [
    "--offload-arch=" + ARCH,
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-I" + os.path.join(ROOT, "include"),
    "-I" + CSRC,
    # Keep the compiler from emitting packed FP32 instructions.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libsuf_hip.so)")


def _deps():
    return glob.glob(os.path.join(CSRC, "*.hpp")) + glob.glob(os.path.join(ROOT, "include", "*.h"))


def _stale(src, obj):
    if not os.path.exists(obj):
        return True
    t = os.path.getmtime(obj)
    return any(os.path.getmtime(p) > t for p in [src] + _deps())


def _compile(args):
    cc, src, obj = args
    tmp = obj + ".tmp"
    cmd = [cc] + HIPCC_FLAGS + ["-c", src, "-o", tmp]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError("hipcc failed for %s:\n%s" % (os.path.basename(src), out))
    os.replace(tmp, obj)
    return out


def build(if_stale=False, jobs=None):
    cc = hipcc()
    os.makedirs(OBJDIR, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.cpp")))
    work = []
    objs = []
    for s in srcs:
        o = os.path.join(OBJDIR, os.path.basename(s) + ".o")
        objs.append(o)
        if not if_stale or _stale(s, o):
            work.append((cc, s, o))
    jobs = jobs or min(8, max(1, os.cpu_count() or 1))
    with ThreadPoolExecutor(jobs) as ex:
        for out in ex.map(_compile, work):
            if out.strip():
                sys.stderr.write(out + "\n")
    if work or not os.path.exists(LIB):
        tmp = LIB + ".tmp"
        cmd = [cc, "--offload-arch=" + ARCH, "-shared", "-fPIC", "-o", tmp] + objs
        r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
        if r.returncode != 0:
            raise RuntimeError("link failed:\n" + r.stdout)
        os.replace(tmp, LIB)
    return LIB


HOST_SRC = os.path.join(PKG, "host")
CPP_TESTS = os.path.join(ROOT, "tests", "cpp")
CPP_TEST_OUT = os.path.join(CPP_TESTS, "_build")


def build_host_tests():
    """Compiles the C++ proto-interface backend (suf_amd/host) into each C++
    test driver under tests/cpp, linked against libsuf_hip.so (g++, no HIP
    headers: the backend reaches the GPU only through the C ABI)."""
    os.makedirs(CPP_TEST_OUT, exist_ok=True)
    host = sorted(glob.glob(os.path.join(HOST_SRC, "*.cpp")))
    outs = []
    for t in sorted(glob.glob(os.path.join(CPP_TESTS, "*.cpp"))):
        exe = os.path.join(CPP_TEST_OUT, os.path.splitext(os.path.basename(t))[0])
        rel = os.path.relpath(LIBDIR, CPP_TEST_OUT)
        cmd = ["g++", "-std=c++17", "-O2", "-Wall", "-Wextra", "-pthread",
               "-I" + os.path.join(ROOT, "include"), t] + host + [
               "-L" + LIBDIR, "-lsuf_hip", "-Wl,-rpath,$ORIGIN/" + rel,
               "-Wl,-rpath-link,/opt/rocm/lib", "-o", exe + ".tmp"]
        r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
        if r.returncode != 0:
            raise RuntimeError("g++ failed for %s:\n%s" % (os.path.basename(t), r.stdout))
        os.replace(exe + ".tmp", exe)
        outs.append(exe)
    return outs


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--if-stale", action="store_true")
    ap.add_argument("-j", type=int, default=None)
    a = ap.parse_args()
    print(build(if_stale=a.if_stale, jobs=a.j))
    for exe in build_host_tests():
        print(exe)


if __name__ == "__main__":
    main()
