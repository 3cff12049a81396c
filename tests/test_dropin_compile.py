"""The drop-in at compile time (CPU): inside the reference's include tree,
  * suf_amd/host/hip_pfss_backend.cpp compiles against SUF's own proto
    headers (SUF_HIP_USE_REFERENCE_PROTO), so HipPfssBackend implements the
    reference's interfaces, not a restatement of them;
  * the launcher shim compiles under SUF's headers too, and one translation
    unit holds the reference's runtime/cuda_primitives.hpp together with the
    replacement include/suf_hip/cuda_primitives.hpp (identical extern "C"
    prototypes, or it fails), calls every launcher with the reference's
    argument types and builds the backend through the replacement factory
    (include/proto/backend_factory.hpp:20-89 plus the hip kind).
Skipped when the reference tree is absent (it never is on this machine's
CPU runs; it is never needed at run time)."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = os.environ.get("SUF_REFERENCE_ROOT", "/root/reference")
REF_INC = os.path.join(REF, "include")


def _gxx(src, extra=()):
    if not os.path.isdir(os.path.join(REF_INC, "proto")):
        pytest.skip("reference include tree not present")
    if not shutil.which("g++"):
        pytest.skip("g++ not available")
    cmd = ["g++", "-std=c++17", "-fsyntax-only", "-Wall", "-Wextra", "-Wno-unused-parameter",
           "-DSUF_HIP_USE_REFERENCE_PROTO", "-I" + os.path.join(ROOT, "include"), "-I" + REF_INC,
           *extra, src]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    assert r.returncode == 0, r.stdout[-4000:]


def test_backend_compiles_against_reference_proto_headers():
    _gxx(os.path.join(ROOT, "suf_amd", "host", "hip_pfss_backend.cpp"))


def test_launcher_shim_compiles_against_reference_headers():
    _gxx(os.path.join(ROOT, "suf_amd", "host", "cuda_primitives_shim.cpp"),
         ["-include", os.path.join(REF_INC, "runtime", "cuda_primitives.hpp")])


def test_reference_tu_with_shim_and_factory_compiles():
    _gxx(os.path.join(ROOT, "tests", "cpp", "dropin", "reference_dropin_tu.cpp"))
