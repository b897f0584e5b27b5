"""The packed kernels' tile orders (smx::tile_of) are bijections from a
launch's workgroups onto its tile grid: a host build of the device function,
run over every grid up to 72 x 72 tiles and every order. A tile that an
order mapped twice or never would leave part of C unwritten; one outside
the grid would read and write out of bounds."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("hipcc") is None, reason="needs hipcc for the host build")
def test_every_tile_order_is_a_bijection(tmp_path):
    exe = tmp_path / "tile_order_check"
    build = subprocess.run(["hipcc", "-O2", "-std=c++17", "-o", str(exe), os.path.join(HERE, "tile_order_check.cpp")],
                           capture_output=True, text=True, timeout=600)
    assert build.returncode == 0, build.stderr[-3000:]
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    assert run.returncode == 0 and run.stdout.startswith("ok"), run.stdout[-2000:]
