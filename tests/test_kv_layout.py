"""Host-side checks of the K/V tile image layout (kv_image.h), compiled from
tests/native/kv_layout_check.cpp: element offsets are a bijection onto the
image, head groups / V dims fill whole lines, and attention's LDS operand
reads are bank-conflict free on 64- and 32-bank LDS."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


def test_kv_image_layout(tmp_path):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    exe = str(tmp_path / "kv_layout_check")
    src = os.path.join(HERE, "native", "kv_layout_check.cpp")
    r = subprocess.run([hipcc, "-O1", "-std=c++17", "-x", "hip", "--offload-arch=gfx950", "-o", exe, src],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    out = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    print(out.stdout)
    assert out.returncode == 0 and out.stdout.strip().endswith("OK"), out.stdout[-2000:]
