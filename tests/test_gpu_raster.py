"""Tile orders of the packed launch (tile_of's spread, chunks and blocks).

The library picks an order per launch from its packed operand sizes, and
SMX_RASTER forces one; the setting is read once per process, so each order
runs in a child process here. The products are of small integers with
float32 output, which both kernels compute exactly whatever their summation
order: every output element must equal the float64 product, so a tile that
an order maps twice or never shows up as a wrong element.
"""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# Tile grids of 128 x 128 product-space tiles (bm = bn = 256): 8 x 13 = 104
# tiles (13 per XCD, all in a partial chunk) and 16 x 20 = 320 (one full
# chunk of 32 and 8 more per XCD), so every branch of the order is taken.
CHILD = r"""
import sys
import torch
import strassen_tpu_amd as smx

dev = torch.device("cuda:0")
gen = torch.Generator().manual_seed(5)
for m, k, n in ((2048, 1024, 3328), (4096, 512, 5120)):
    a = torch.randint(-3, 4, (m, k), generator=gen).to(torch.float64)
    b = torch.randint(-3, 4, (k, n), generator=gen).to(torch.float64)
    want = a @ b
    a_dev = a.to(torch.bfloat16).to(dev)
    w_dev = b.to(torch.bfloat16).t().contiguous().to(dev).t()
    for name, fn, layout in (("strassen", smx.strassen_matmul, smx.strassen_weight_layout),
                             ("cubic", smx.cubic_matmul, smx.cubic_weight_layout)):
        got = fn(a_dev, layout(w_dev, 256, 512), bm=256, bn=256, bk=512, output_dtype=torch.float32)
        bad = int((got.double().cpu() != want).sum())
        print(f"{name} {m}x{k}x{n}: {bad} wrong elements", flush=True)
        if bad:
            sys.exit(1)
print("ok", flush=True)
"""


@pytest.mark.parametrize("order", ["spread", "chunks", "blocks"])
def test_every_tile_order_computes_every_tile_once(order):
    env = dict(os.environ, SMX_RASTER=order, PYTHONPATH=REPO + os.pathsep + os.environ.get("PYTHONPATH", ""))
    print(f"SMX_RASTER={order}", flush=True)
    run = subprocess.run([sys.executable, "-c", CHILD], env=env, cwd=REPO, capture_output=True, text=True,
                         timeout=300)
    print(run.stdout, run.stderr[-2000:], flush=True)
    assert run.returncode == 0 and run.stdout.strip().endswith("ok"), run.stdout + run.stderr[-2000:]
