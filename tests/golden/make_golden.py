"""Write the small golden fixtures under tests/golden/ from the CPU oracle.

Run from the repository root:  python tests/golden/make_golden.py

Fixtures (numpy .npz, no pickles):
  e4m3_tables.npz  enc_bf16[65536] u8: torch's e4m3fn cast of every bf16 bit
                   pattern; dec[256] f32: torch's decode of every code.
  kv_small.npz     a ragged 40-token, 2-head, head_dim-128 K/V pair packed into
                   a 5-page pool of 16-token pages through a shuffled page
                   table; inputs as bf16 bit patterns, pool codes and scales.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import fp8 as ofp8  # noqa: E402
from oracle import kv as okv  # noqa: E402
from waveforcing_amd import inputs  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))


def e4m3_tables() -> None:
    allbf = ofp8.all_bf16_as_f32()
    enc = ofp8.encode(allbf).numpy().copy()
    dec = ofp8.decode(torch.arange(256, dtype=torch.int32).to(torch.uint8)).numpy().copy()
    np.savez(os.path.join(OUT, "e4m3_tables.npz"), enc_bf16=enc, dec=dec)


def kv_small() -> None:
    T, H, D, page, pool_pages = 40, 2, 128, 16, 5
    k = inputs.heavy_tailed_kv(T, H, D, seed=11)
    v = inputs.heavy_tailed_kv(T, H, D, seed=12)
    # A few exact-tie and extreme rows: zeros, a single spike, values that
    # quantize to exact e4m3 midpoints.
    k[0] = 0
    k[1, 0] = 0
    k[1, 0, 5] = 3.0
    v[2, 1] = torch.linspace(-448, 448, D).to(torch.bfloat16)
    table = [3, 0, 4]
    kc, ks = okv.new_pool(pool_pages, page, H, D)
    vc, vs = okv.new_pool(pool_pages, page, H, D)
    okv.pack(k, table, page, kc, ks)
    okv.pack(v, table, page, vc, vs)
    np.savez(
        os.path.join(OUT, "kv_small.npz"),
        k_bits=k.view(torch.int16).numpy(), v_bits=v.view(torch.int16).numpy(),
        table=np.array(table, dtype=np.int32), page_tokens=np.int32(page), pool_pages=np.int32(pool_pages),
        k_codes=kc.numpy(), k_scales=ks.numpy(), v_codes=vc.numpy(), v_scales=vs.numpy(),
    )


if __name__ == "__main__":
    e4m3_tables()
    kv_small()
    for f in sorted(os.listdir(OUT)):
        print(f, os.path.getsize(os.path.join(OUT, f)))
