"""Wan DiT block weights on disk: the diffusers key layout, and offline W8A8 packing.

Layouts of one block's 27 tensors (BlockParams):

* ``diffusers``: the CausalWanTransformer3DModel layout the reference ships its
  checkpoint in, ``blocks.{i}.attn1.to_q.weight`` ... (the renames of
  scripts/convert_rf_ckpt_to_diffusers.py:26-75);
* ``raw``: the RollingForcing / naive_rt module names the conversion starts
  from, ``blocks.{i}.self_attn.q.weight`` ... (with or without the FSDP
  ``model._fsdp_wrapped_module.`` prefix).

:func:`load_block_params` reads one block from a ``.safetensors`` file, a
directory holding one, or a sharded ``*.safetensors.index.json``, touching
only that block's tensors (memory-mapped reads).

Offline packing replaces the load-then-swap of the reference
(wave_rt/runtime/backend.py:303-314, where every linear is re-quantized after
the bf16 weights load): :func:`pack_block` quantizes a block's linears once
with the HIP per-channel int8 quantizer and :func:`save_packed` writes int8
weights, fp32 per-channel scales, bf16 biases and the block's other bf16
tensors as safetensors; :func:`load_packed` + ``QuantizedWanBlock.from_packed``
put them on the GPU without quantizing again.
"""

from __future__ import annotations

import json
import os
from dataclasses import fields

import torch
from safetensors import safe_open
from safetensors.torch import save_file

from .block import BlockParams

FSDP_PREFIX = "model._fsdp_wrapped_module."
PACKED_FORMAT = "waveforcing_amd.w8a8.v1"

# BlockParams field -> (diffusers submodule, raw submodule, tensor).  The
# submodule renames are the checkpoint format (convert_rf_ckpt_to_diffusers.py:26-43).
_FIELDS = {
    "modulation": ("scale_shift_table", "modulation", None),
    "q_w": ("attn1.to_q", "self_attn.q", "weight"), "q_b": ("attn1.to_q", "self_attn.q", "bias"),
    "k_w": ("attn1.to_k", "self_attn.k", "weight"), "k_b": ("attn1.to_k", "self_attn.k", "bias"),
    "v_w": ("attn1.to_v", "self_attn.v", "weight"), "v_b": ("attn1.to_v", "self_attn.v", "bias"),
    "o_w": ("attn1.to_out.0", "self_attn.o", "weight"), "o_b": ("attn1.to_out.0", "self_attn.o", "bias"),
    "norm_q": ("attn1.norm_q", "self_attn.norm_q", "weight"),
    "norm_k": ("attn1.norm_k", "self_attn.norm_k", "weight"),
    "norm3_w": ("norm2", "norm3", "weight"), "norm3_b": ("norm2", "norm3", "bias"),
    "cq_w": ("attn2.to_q", "cross_attn.q", "weight"), "cq_b": ("attn2.to_q", "cross_attn.q", "bias"),
    "ck_w": ("attn2.to_k", "cross_attn.k", "weight"), "ck_b": ("attn2.to_k", "cross_attn.k", "bias"),
    "cv_w": ("attn2.to_v", "cross_attn.v", "weight"), "cv_b": ("attn2.to_v", "cross_attn.v", "bias"),
    "co_w": ("attn2.to_out.0", "cross_attn.o", "weight"), "co_b": ("attn2.to_out.0", "cross_attn.o", "bias"),
    "cnorm_q": ("attn2.norm_q", "cross_attn.norm_q", "weight"),
    "cnorm_k": ("attn2.norm_k", "cross_attn.norm_k", "weight"),
    "fc_in_w": ("ffn.net.0.proj", "ffn.0", "weight"), "fc_in_b": ("ffn.net.0.proj", "ffn.0", "bias"),
    "fc_out_w": ("ffn.net.2", "ffn.2", "weight"), "fc_out_b": ("ffn.net.2", "ffn.2", "bias"),
}
assert set(_FIELDS) == {f.name for f in fields(BlockParams)}

# The block linears the W8A8 swap quantizes (scope "all", wave_rt/runtime/fp8.py:93-137).
LINEARS = ("q", "k", "v", "o", "cq", "ck", "cv", "co", "fc_in", "fc_out")


def block_key(block: int, field: str, layout: str = "diffusers") -> str:
    """Checkpoint key of a BlockParams field of block ``block``."""
    dif, raw, tensor = _FIELDS[field]
    if layout == "diffusers":
        sub = dif
    elif layout == "raw":
        sub = raw
    else:
        raise ValueError(f"unknown layout {layout!r} (diffusers or raw)")
    return f"blocks.{block}.{sub}" + (f".{tensor}" if tensor else "")


class _Tensors:
    """Key -> tensor reads over one safetensors file or a sharded index (memory-mapped)."""

    def __init__(self, path: str) -> None:
        if os.path.isdir(path):
            idx = [f for f in os.listdir(path) if f.endswith(".safetensors.index.json")]
            single = [f for f in os.listdir(path) if f.endswith(".safetensors")]
            if idx:
                path = os.path.join(path, sorted(idx)[0])
            elif len(single) == 1:
                path = os.path.join(path, single[0])
            else:
                raise FileNotFoundError(f"{path}: no safetensors index and {len(single)} safetensors files")
        if path.endswith(".index.json"):
            with open(path) as f:
                weight_map = json.load(f)["weight_map"]
            base = os.path.dirname(path)
            self._where = {k: os.path.join(base, v) for k, v in weight_map.items()}
        else:
            with safe_open(path, framework="pt") as f:
                self._where = {k: path for k in f.keys()}
        self._open: dict = {}

    def keys(self):
        return self._where.keys()

    def get(self, key: str) -> torch.Tensor:
        path = self._where.get(key)
        if path is None:
            raise KeyError(f"checkpoint has no tensor {key!r}")
        f = self._open.get(path)
        if f is None:
            f = self._open[path] = safe_open(path, framework="pt")
        return f.get_tensor(key)


def _detect_layout(keys, block: int) -> tuple[str, str]:
    """(layout, key prefix) of a checkpoint, from block ``block``'s q weight."""
    keys = set(keys)
    for layout in ("diffusers", "raw"):
        k = block_key(block, "q_w", layout)
        for prefix in ("", FSDP_PREFIX):
            if prefix + k in keys:
                return layout, prefix
    raise KeyError(f"block {block}: neither the diffusers nor the raw layout found "
                   f"(looked for {block_key(block, 'q_w')!r} and {block_key(block, 'q_w', 'raw')!r})")


def load_block_params(path: str, block: int, layout: str | None = None) -> BlockParams:
    """One block's bf16 parameters (CPU) from a checkpoint in either layout."""
    src = _Tensors(path)
    if layout is None:
        layout, prefix = _detect_layout(src.keys(), block)
    else:
        prefix = FSDP_PREFIX if (FSDP_PREFIX + block_key(block, "q_w", layout)) in src.keys() else ""
    out = {name: src.get(prefix + block_key(block, name, layout)).to(torch.bfloat16) for name in _FIELDS}
    p = BlockParams(**out)
    _check_shapes(p, block)
    return p


def _check_shapes(p: BlockParams, block: int) -> None:
    dim = p.q_w.shape[1]
    ffn = p.fc_in_w.shape[0]
    want = {
        "modulation": (1, 6, dim), "fc_in_w": (ffn, dim), "fc_in_b": (ffn,), "fc_out_w": (dim, ffn),
        "fc_out_b": (dim,),
    }
    for f in fields(p):
        t = getattr(p, f.name)
        if f.name in want:
            shape = want[f.name]
        elif f.name.endswith("_w") and f.name not in ("norm3_w",):
            shape = (dim, dim)
        else:
            shape = (dim,)
        if tuple(t.shape) != shape:
            raise ValueError(f"block {block}: {f.name} has shape {tuple(t.shape)}, expected {shape}")


def save_block_params(path: str, blocks: dict[int, BlockParams], layout: str = "diffusers") -> None:
    """Write blocks' bf16 parameters under the given layout (one safetensors file)."""
    out = {}
    for i, p in blocks.items():
        for name in _FIELDS:
            out[block_key(i, name, layout)] = getattr(p, name).to(torch.bfloat16).contiguous().cpu()
    save_file(out, path)


# --------------------------------------------------------------- W8A8 packing
def _linear_fields(lin: str) -> tuple[str, str]:
    return f"{lin}_w", f"{lin}_b"


def pack_block(p: BlockParams, device="cuda") -> dict[str, torch.Tensor]:
    """Per-channel int8 weights (HIP quantizer) + fp32 scales for the block's linears, plus its
    other tensors in bf16.  Keys are BlockParams names; linears get ``{lin}_i8`` / ``{lin}_scale``."""
    from .fp8 import _quant_rows_i8

    out: dict[str, torch.Tensor] = {}
    for lin in LINEARS:
        wf, bf = _linear_fields(lin)
        q, s = _quant_rows_i8(getattr(p, wf).to(device).contiguous())
        out[f"{lin}_i8"] = q.cpu()
        out[f"{lin}_scale"] = s.cpu()
        out[bf] = getattr(p, bf).to(torch.bfloat16).cpu()
    linear_weights = {_linear_fields(lin)[0] for lin in LINEARS}
    for name in _FIELDS:
        if name not in out and name not in linear_weights:
            out[name] = getattr(p, name).to(torch.bfloat16).cpu()
    return out


def save_packed(path: str, packed: dict[int, dict[str, torch.Tensor]]) -> None:
    """Write packed blocks (from :func:`pack_block`) to one safetensors file."""
    out = {f"blocks.{i}.{k}": v.contiguous() for i, d in packed.items() for k, v in d.items()}
    save_file(out, path, metadata={"format": PACKED_FORMAT})


def load_packed(path: str, block: int) -> dict[str, torch.Tensor]:
    """One packed block (CPU tensors) from a file written by :func:`save_packed`."""
    with safe_open(path, framework="pt") as f:
        meta = f.metadata() or {}
        if meta.get("format") != PACKED_FORMAT:
            raise ValueError(f"{path}: not a {PACKED_FORMAT} file (format={meta.get('format')!r})")
        pre = f"blocks.{block}."
        keys = [k for k in f.keys() if k.startswith(pre)]
        if not keys:
            raise KeyError(f"{path}: no block {block}")
        d = {k[len(pre):]: f.get_tensor(k) for k in keys}
    missing = [f"{lin}_{s}" for lin in LINEARS for s in ("i8", "scale")
               if f"{lin}_{s}" not in d]
    if missing:
        raise KeyError(f"{path}: block {block} lacks {missing}")
    return d
