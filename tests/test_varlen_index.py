"""The packed-sequence (cu_seqlens) index arithmetic of the kernels, compiled on the host.

csrc/varlen_index.h holds the clamped offsets and the slot mapping that the chunk prep and scan kernels, the
single-launch chunk kernel, the attention kernel and the short convolution read cu_seqlens through.  The offsets
are device-resident, so the library cannot check them on the host without a synchronisation; the kernels clamp
them instead.  This test builds varlen_index_check.cpp against that header with g++ and runs it: for valid offsets
and for offsets that break the contract, every slot and row the mappings yield stays inside the launch's slots and
the sequence's rows, and for valid offsets the prep's slot -> (sequence, chunk) map and the scan's (sequence,
chunk) -> slot map agree one to one.  No GPU is involved.
"""

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(HERE), "gtar-kimik3-public_amd", "csrc")


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_varlen_index_in_bounds(tmp_path):
    exe = str(tmp_path / "varlen_index_check")
    subprocess.run(["g++", "-O1", "-std=c++17", "-Wall", "-I", CSRC, os.path.join(HERE, "varlen_index_check.cpp"),
                    "-o", exe], check=True)
    res = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(res.stdout)
    assert res.returncode == 0 and res.stdout.startswith("ok"), res.stdout + res.stderr
