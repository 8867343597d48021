"""The C ABI from plain C on the GPU: tests/c_abi/abi_check.c runs the reference's known
answers (flat.rs:323-338, 370-383), the inner-product padding, the raw keys of the CUDA seam
(gpu.rs:10-15, knn.cu:123-180), an explicit-codebook PQ search and the error codes."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu


def test_c_program_on_gpu(gpu):
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c_abi", "abi_check")
    assert os.path.exists(path), "build tests/c_abi first (__graft_entry__.build())"
    out = subprocess.run([path], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    assert out.stdout.startswith("abi_check ok (gfx950 path")
