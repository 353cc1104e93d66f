"""Checkpoint layouts on the CPU (no GPU): one block's 27 tensors under the
diffusers keys of scripts/convert_rf_ckpt_to_diffusers.py:26-75 and under the
raw RollingForcing names (with and without the FSDP prefix), single file,
directory and sharded index; errors for missing blocks and wrong shapes."""

import json
import os

import pytest
import torch
from safetensors.torch import save_file

from waveforcing_amd import checkpoint as ck
from waveforcing_amd.block import BlockParams, random_block_params

DIM, FFN = 64, 160


def _same(a: BlockParams, b: BlockParams):
    for name in ck._FIELDS:
        assert torch.equal(getattr(a, name), getattr(b, name)), name


def test_block_keys_follow_the_diffusers_renames():
    # spot checks of the published layout (per block: attn1/attn2 q,k,v,out.0, norms, ffn.net.0.proj/2)
    assert ck.block_key(3, "q_w") == "blocks.3.attn1.to_q.weight"
    assert ck.block_key(3, "co_b") == "blocks.3.attn2.to_out.0.bias"
    assert ck.block_key(0, "norm3_w") == "blocks.0.norm2.weight"
    assert ck.block_key(0, "fc_in_w") == "blocks.0.ffn.net.0.proj.weight"
    assert ck.block_key(0, "modulation") == "blocks.0.scale_shift_table"
    assert ck.block_key(5, "fc_out_b", "raw") == "blocks.5.ffn.2.bias"
    assert ck.block_key(5, "norm3_b", "raw") == "blocks.5.norm3.bias"
    # 27 tensors per block: 30 blocks + 15 top-level tensors = the 825 keys of the 1.3B checkpoint
    assert len(ck._FIELDS) == 27 and 30 * 27 + 15 == 825
    keys = {ck.block_key(0, n) for n in ck._FIELDS}
    assert len(keys) == 27


@pytest.mark.parametrize("layout", ["diffusers", "raw"])
def test_roundtrip_single_file(tmp_path, layout):
    blocks = {0: random_block_params(DIM, FFN, seed=1), 1: random_block_params(DIM, FFN, seed=2)}
    path = str(tmp_path / "m.safetensors")
    ck.save_block_params(path, blocks, layout)
    for i, p in blocks.items():
        _same(ck.load_block_params(path, i), p)
        _same(ck.load_block_params(str(tmp_path), i, layout), p)


def test_fsdp_prefixed_raw_and_sharded_index(tmp_path):
    p0, p1 = random_block_params(DIM, FFN, seed=3), random_block_params(DIM, FFN, seed=4)
    raw = {ck.FSDP_PREFIX + ck.block_key(0, n, "raw"): getattr(p0, n).contiguous() for n in ck._FIELDS}
    save_file(raw, str(tmp_path / "raw.safetensors"))
    _same(ck.load_block_params(str(tmp_path / "raw.safetensors"), 0), p0)
    # two shards split by block, plus the index
    shard = tmp_path / "sharded"
    shard.mkdir()
    wm = {}
    for i, p in ((0, p0), (1, p1)):
        name = f"diffusion_pytorch_model-0000{i + 1}-of-00002.safetensors"
        d = {ck.block_key(i, n): getattr(p, n).contiguous() for n in ck._FIELDS}
        save_file(d, str(shard / name))
        wm.update({k: name for k in d})
    with open(shard / "diffusion_pytorch_model.safetensors.index.json", "w") as f:
        json.dump({"metadata": {}, "weight_map": wm}, f)
    _same(ck.load_block_params(str(shard), 1), p1)
    _same(ck.load_block_params(str(shard), 0), p0)


def test_missing_block_and_bad_shape(tmp_path):
    p = random_block_params(DIM, FFN, seed=5)
    path = str(tmp_path / "m.safetensors")
    ck.save_block_params(path, {0: p})
    with pytest.raises(KeyError, match="block 7"):
        ck.load_block_params(path, 7)
    bad = {ck.block_key(0, n): getattr(p, n).contiguous() for n in ck._FIELDS}
    bad[ck.block_key(0, "o_w")] = torch.zeros((DIM, DIM + 8), dtype=torch.bfloat16)
    save_file(bad, str(tmp_path / "bad.safetensors"))
    with pytest.raises(ValueError, match="o_w"):
        ck.load_block_params(str(tmp_path / "bad.safetensors"), 0)


def test_packed_file_is_checked(tmp_path):
    save_file({"blocks.0.q_i8": torch.zeros((4, 16), dtype=torch.int8)}, str(tmp_path / "x.safetensors"))
    with pytest.raises(ValueError, match="not a"):
        ck.load_packed(str(tmp_path / "x.safetensors"), 0)
    save_file({"blocks.0.q_i8": torch.zeros((4, 16), dtype=torch.int8)}, str(tmp_path / "y.safetensors"),
              metadata={"format": ck.PACKED_FORMAT})
    with pytest.raises(KeyError, match="lacks"):
        ck.load_packed(str(tmp_path / "y.safetensors"), 0)
