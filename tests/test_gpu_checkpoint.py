"""GPU check of offline W8A8 packing: a block written in the diffusers layout,
loaded, packed once with the HIP quantizer, saved, loaded back and built with
QuantizedWanBlock.from_packed runs bit-for-bit like the block built directly
from the bf16 parameters (which quantizes at construction); the packed int8
weights and scales equal the oracle's per-channel quantization."""

import pytest
import torch

from oracle import linear as olin
from waveforcing_amd import checkpoint as ck
from waveforcing_amd import rope
from waveforcing_amd.block import QuantizedWanBlock, random_block_params
from waveforcing_amd.kv import Fp8PagePool

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _forward(blk, x, e, heads, frames, h, w, context, seed):
    T = x.shape[0]
    page = h * w
    g = torch.Generator().manual_seed(seed)
    prior = torch.randn((T, heads, 128), generator=g).to(torch.bfloat16).to(DEV)
    pool = Fp8PagePool(2 * frames, heads, 128, page, DEV)
    pool.pack(prior, prior, pool.page_table(list(range(frames))))
    cos, sin = rope.cos_sin(frames, h, w, frames, device=DEV)
    tkv = blk.text_kv(context)
    y = x.clone()
    blk.forward(y, e, cos, sin, pool, pool.page_table(list(range(2 * frames))),
                pool.page_table(list(range(frames, 2 * frames))), 2 * T, tkv)
    return y, pool


def test_packed_block_equals_direct_block(tmp_path):
    dim, heads, ffn = 256, 2, 512
    frames, h, w = 3, 8, 8
    params = random_block_params(dim, ffn, seed=11)
    src = str(tmp_path / "model.safetensors")
    ck.save_block_params(src, {4: params})
    loaded = ck.load_block_params(src, 4)
    packed = ck.pack_block(loaded, DEV)
    for lin in ck.LINEARS:
        oq, os_ = olin.i8_quant_rows(getattr(params, f"{lin}_w"))
        assert torch.equal(packed[f"{lin}_i8"], oq) and torch.equal(packed[f"{lin}_scale"], os_), lin
    out = str(tmp_path / "w8a8.safetensors")
    ck.save_packed(out, {4: packed})
    blk_p = QuantizedWanBlock.from_packed(ck.load_packed(out, 4), heads, DEV)
    blk_d = QuantizedWanBlock(params, heads, DEV)
    g = torch.Generator().manual_seed(12)
    T = frames * h * w
    x = torch.randn((T, dim), generator=g).to(torch.bfloat16).to(DEV)
    e = (torch.randn((frames, 6, dim), generator=g) * 0.1).to(torch.bfloat16).to(DEV)
    context = torch.randn((32, dim), generator=g).to(torch.bfloat16).to(DEV)
    y_p, pool_p = _forward(blk_p, x, e, heads, frames, h, w, context, 13)
    y_d, pool_d = _forward(blk_d, x, e, heads, frames, h, w, context, 13)
    assert torch.equal(y_p, y_d)
    assert torch.equal(pool_p.k_codes, pool_d.k_codes) and torch.equal(pool_p.v_scales, pool_d.v_scales)
