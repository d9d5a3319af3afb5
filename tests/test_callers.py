"""Compiled callers of the boundary: a C program over the cuvsOctex* ABI and a C++ program over the
cuvs::neighbors::octex API (tests/c/), built with gcc / g++ against include/ and liboctex_amd.so as a C or C++ user
of the reference would build theirs (examples/c/search.c, examples/cpp/search.cu).  Compiling runs on the CPU; the
GPU test runs both, build -> load -> search, and checks their results against the Python package's."""

import os
import subprocess

import numpy as np
import pytest
from conftest import ROOT, clustered, exact_knn, recall

from octex_amd import _lib

SRC = os.path.join(ROOT, "tests", "c")
LIBDIR = os.path.dirname(_lib.LIB_PATH)
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")


def compile_callers(out):
    """The C and C++ callers linked against the library (the C++ one also against the HIP runtime, which its
    raft::resources calls)."""
    c, cpp = os.path.join(out, "octex_search_c"), os.path.join(out, "octex_search_cpp")
    link = ["-L", LIBDIR, "-loctex_amd", f"-Wl,-rpath,{LIBDIR}"]
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"),
                    os.path.join(SRC, "octex_search.c"), "-o", c] + link, check=True)
    subprocess.run(["g++", "-std=c++17", "-Wall", "-Werror", "-D__HIP_PLATFORM_AMD__", "-I",
                    os.path.join(ROOT, "include"), "-I", os.path.join(ROCM, "include"),
                    os.path.join(SRC, "octex_search.cpp"), "-o", cpp] + link
                   + ["-L", os.path.join(ROCM, "lib"), "-lamdhip64", f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}"],
                   check=True)
    return c, cpp


@pytest.mark.skipif(not os.path.isfile(_lib.LIB_PATH), reason="the library is not built")
def test_callers_compile(tmp_path):
    for exe in compile_callers(str(tmp_path)):
        out = subprocess.run([exe], capture_output=True, text=True)
        assert out.returncode == 2 and "usage" in out.stderr


@pytest.mark.gpu
def test_callers_match_python(tmp_path):
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import octex_amd

    X, Q = clustered(n=5000, m=64, d=32, clusters=12, seed=11)
    k = 10
    X.tofile(tmp_path / "x.f32")
    Q.tofile(tmp_path / "q.f32")
    gt, _ = exact_knn(X.astype(np.float16).astype(np.float32), Q)
    results = []
    for exe, name in zip(compile_callers(str(tmp_path)), ("c", "cpp")):
        d = tmp_path / f"index_{name}"
        out = tmp_path / f"out_{name}"
        run = subprocess.run([exe, str(d), str(len(X)), str(X.shape[1]), str(len(Q)), str(k), str(tmp_path / "x.f32"),
                              str(tmp_path / "q.f32"), str(out)], capture_output=True, text=True, timeout=120)
        assert run.returncode == 0, run.stderr
        I = np.fromfile(f"{out}.i64", np.int64).reshape(len(Q), k)
        D = np.fromfile(f"{out}.f32", np.float32).reshape(len(Q), k)
        Dp, Ip = octex_amd.load(d).search(Q, k=k, read=16, starts=64, waves=2)
        assert np.array_equal(I, Ip) and np.array_equal(D, Dp)
        assert recall(I, gt) >= 0.95
        results.append((I, D))
    assert np.array_equal(results[0][0], results[1][0]) and np.array_equal(results[0][1], results[1][1])
