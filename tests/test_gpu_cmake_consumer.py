"""The downstream C++ program built against the installed CMake package
(tests/cmake_consumer/consumer.cpp via find_package(bitsqz_llm CONFIG)) runs
on the GPU; the packed objects and decoded matrices it writes are checked
against the oracle like every other ABI test: the reference walkthrough's
8 x 8 case (examples/bitsqz_llm_walkthrough.cpp:34-121) section by section,
and a direct NF4_DQ case with outliers and error top-k byte for byte."""
import os
import subprocess

import numpy as np
import pytest

import bitsqz_amd as B
from oracle import oracle as O
from _svdcase import check_sections

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CONSUMER = os.path.join(ROOT, "tests", "cmake_consumer", "_build", "bsq_consumer")


def test_installed_package_consumer(tmp_path):
    r = subprocess.run([CONSUMER, str(tmp_path)], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stderr
    assert "consumer: ok" in r.stdout
    # walkthrough: 8 x 8 host input, rank 4, NF4 U/V and S
    i = np.arange(64)
    x = ((i % 8) * np.float32(0.25) + (i // 8) * np.float32(0.5)).astype(np.float32).reshape(8, 8)
    data = (tmp_path / "walk_packed.bin").read_bytes()
    out = np.fromfile(tmp_path / "walk_decoded.bin", np.float32).reshape(8, 8)
    check_sections(x, data, out, 0.0, 0.0, 4, B.NF4, B.NF4)
    # direct: NF4_DQ + outlier 0.01 + error 0.02 on 64 x 512, device input
    xd = np.fromfile(tmp_path / "direct_input.bin", np.float32).reshape(64, 512)
    pd = (tmp_path / "direct_packed.bin").read_bytes()
    od = np.fromfile(tmp_path / "direct_decoded.bin", np.float32).reshape(64, 512)
    ref = O.compress(xd, O.Config(64, 512, outlier_ratio=0.01, error_ratio=0.02, svd_niters=1,
                                  direct_format=O.NF4_DQ))
    assert ref.flags == (O.FLAG_OUTLIER | O.FLAG_ERROR)
    assert O.mask_pointer(pd) == O.mask_pointer(ref.to_bytes())
    assert od.tobytes() == O.decompress(ref).tobytes()
