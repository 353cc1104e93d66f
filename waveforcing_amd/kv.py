"""FP8 e4m3fn paged KV pool on one GPU.

The reference keeps per-(generation, layer) bf16 slabs of shape
``(GT, Ln, Wmax*T, H, D)`` and fills fixed slots with DMA copies
(wave_rt/denoiser/exchange/paged.py:43-48,120-145).  Its FP8 KV modes quantize
per tensor (common.py:143-164) or cast without a scale (onesided.py:151-154),
and paged mode rejects FP8 (paged.py:31-32).

Here the slabs become one pool of physical pages per tensor (K and V), each
page one latent frame of ``page_tokens`` tokens, stored as e4m3fn codes with
one fp32 scale per (token, head):

    codes  uint8   [pool_pages, page_tokens, H, D]
    scales float32 [pool_pages, H, page_tokens]

A logical token sequence (one layer's context) is a list of physical page
ids.  With the identity page table and contiguous pages, page ``p`` holds
slab rows ``[p*page_tokens, (p+1)*page_tokens)`` of the reference layout.
The pool is allocated by the caller (like the reference's ``torch.zeros``
slabs); the HIP kernels never allocate.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Sequence

import torch

from . import _lib, settings


class PageTable:
    """Validated page ids of one logical sequence, on host and device."""

    def __init__(self, ids: Sequence[int], pool_pages: int, device) -> None:
        host = [int(i) for i in ids]
        for i in host:
            if i < 0 or i >= pool_pages:
                raise RuntimeError(f"page id {i} outside pool of {pool_pages} pages")
        self.host = host
        self.pool_pages = pool_pages
        self.dev = torch.tensor(host, dtype=torch.int32, device=device)

    @property
    def dev_ptr(self) -> int:
        return self.dev.data_ptr()

    def __len__(self) -> int:
        return len(self.host)


def _as_thd(x: torch.Tensor, name: str):
    """Accept [T, H, D] or the reference's [1, T, H, D] views (paged.py:207-208) and return
    (tensor, address, (T, H, D), token stride) of the data the kernels read.

    Heads and head_dim must be dense; the token stride may be larger (e.g. a
    column slice of a fused QKV output) as long as it is a multiple of 8.
    Anything else is copied dense first.  No view is made on the fast path.
    """
    shape = x.shape
    strides = x.stride()
    if len(shape) == 4:
        if shape[0] != 1:
            raise ValueError(f"{name}: batch dimension must be 1, got {tuple(shape)}")
        shape, strides = shape[1:], strides[1:]
    if len(shape) != 3:
        raise ValueError(f"{name}: expected [T, H, D], got {tuple(shape)}")
    if x.dtype != torch.bfloat16:
        raise ValueError(f"{name}: expected bfloat16, got {x.dtype}")
    T, H, D = shape
    s0, s1, s2 = strides
    addr = x.data_ptr()
    if s2 != 1 or s1 != D or s0 % 8 or addr % 16 or (T > 1 and s0 < H * D):
        x = x.reshape(T, H, D).contiguous()
        addr, s0 = x.data_ptr(), H * D
    return x, addr, (T, H, D), (s0 if T > 1 else H * D)


def _rope_tables(rope, T: int, D: int, device, tiled: bool = False):
    """Validated (cos, sin) fp32 [R, D/2]: R = T, or with ``tiled`` any R dividing T (token t uses row t % R)."""
    cos, sin = rope
    R = cos.shape[0] if tiled and cos.dim() == 2 else T
    if tiled and (R < 1 or T % R):
        raise ValueError(f"a tiled rope table of {R} rows must divide the {T} tokens")
    for name, t in (("cos", cos), ("sin", sin)):
        on_device = t.device.type == device.type and (device.index is None or t.device.index == device.index)
        if t.dtype != torch.float32 or tuple(t.shape) != (R, D // 2) or not t.is_contiguous() or not on_device:
            raise ValueError(f"rope {name} must be contiguous fp32 [{R}, {D // 2}] on {device}")
    return cos, sin


class Fp8PagePool:
    """K and V page pools in HBM with pack / gather-dequant through the HIP kernels."""

    def __init__(
        self,
        pool_pages: int,
        n_heads: int,
        head_dim: int = settings.HEAD_DIM,
        page_tokens: int = settings.PAGE_TOKENS,
        device="cuda",
    ) -> None:
        if head_dim != 128:
            raise ValueError(f"head_dim={head_dim} unsupported (kernels are specialised for 128)")
        self.pool_pages = pool_pages
        self.n_heads = n_heads
        self.head_dim = head_dim
        self.page_tokens = page_tokens
        self.device = torch.device(device)
        shape_c = (pool_pages, page_tokens, n_heads, head_dim)
        shape_s = (pool_pages, n_heads, page_tokens)
        self.k_codes = torch.zeros(shape_c, dtype=torch.uint8, device=self.device)
        self.v_codes = torch.zeros(shape_c, dtype=torch.uint8, device=self.device)
        self.k_scales = torch.zeros(shape_s, dtype=torch.float32, device=self.device)
        self.v_scales = torch.zeros(shape_s, dtype=torch.float32, device=self.device)
        self._cache_ptrs()

    def _cache_ptrs(self) -> None:
        # device addresses of the four arrays, read by every launch
        self._k_codes_p, self._v_codes_p = self.k_codes.data_ptr(), self.v_codes.data_ptr()
        self._k_scales_p, self._v_scales_p = self.k_scales.data_ptr(), self.v_scales.data_ptr()

    @classmethod
    def view_of(cls, base: "Fp8PagePool", first_page: int, n_pages: int) -> "Fp8PagePool":
        """Pages [first_page, first_page + n_pages) of ``base`` as a pool of their own (shared storage,
        page ids relative to first_page)."""
        if first_page < 0 or n_pages < 1 or first_page + n_pages > base.pool_pages:
            raise ValueError(f"pages [{first_page}, {first_page + n_pages}) outside a pool of {base.pool_pages}")
        self = cls.__new__(cls)
        self.pool_pages = n_pages
        self.n_heads = base.n_heads
        self.head_dim = base.head_dim
        self.page_tokens = base.page_tokens
        self.device = base.device
        sl = slice(first_page, first_page + n_pages)
        self.k_codes, self.v_codes = base.k_codes[sl], base.v_codes[sl]
        self.k_scales, self.v_scales = base.k_scales[sl], base.v_scales[sl]
        self._cache_ptrs()
        return self

    @staticmethod
    def bytes_for(pool_pages: int, n_heads: int, head_dim: int, page_tokens: int) -> int:
        """Device bytes of a pool (K and V codes + scales)."""
        return 2 * pool_pages * page_tokens * n_heads * (head_dim + 4)

    @property
    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.k_codes, self.v_codes, self.k_scales, self.v_scales))

    def page_table(self, ids: Sequence[int]) -> PageTable:
        return PageTable(ids, self.pool_pages, self.device)

    def pages_for(self, n_tokens: int) -> int:
        return -(-n_tokens // self.page_tokens)

    def pack(self, k: torch.Tensor, v: torch.Tensor | None, table: PageTable,
             rope: tuple[torch.Tensor, torch.Tensor] | None = None, tiled: bool = False) -> None:
        """Quantize K (and V) [T, H, D] bf16 into the pages listed by ``table``.

        With ``rope = (cos, sin)`` (fp32 [T, D/2]), K is rotated first and the
        rotated bf16 values are quantized: the anchor re-RoPE plus slot copy of
        _anchor_working (wave_rt/denoiser/exchange/common.py:70-91,
        paged.py:222-227) in one kernel.  With ``tiled``, the tables may have
        R rows for any R dividing T and token t uses row t % R (a batch of equal
        chunks, e.g. every layer's anchor, in one launch).
        """
        kt, kp, shape, ld = _as_thd(k, "k")
        vt, vp = None, None
        if v is not None:
            vt, vp, vshape, vld = _as_thd(v, "v")
            if vshape != shape:
                raise ValueError(f"k {tuple(shape)} and v {tuple(vshape)} differ")
            if vld != ld:
                # one token stride serves K and V; if they differ, pack from dense copies
                kt, vt = kt.reshape(shape).contiguous(), vt.reshape(shape).contiguous()
                kp, vp, ld = kt.data_ptr(), vt.data_ptr(), shape[1] * shape[2]
        T, H, D = shape
        if H != self.n_heads or D != self.head_dim:
            raise ValueError(f"k has H={H}, D={D}; pool has H={self.n_heads}, D={self.head_dim}")
        if len(table) * self.page_tokens < T:
            raise RuntimeError(f"page table of {len(table)} pages cannot hold {T} tokens")
        pool_args = (table.dev_ptr, len(table), self.page_tokens, self._k_codes_p, self._v_codes_p if vp else None,
                     self._k_scales_p, self._v_scales_p if vp else None, self.pool_pages,
                     _lib.stream_handle(self.device))
        if rope is not None:
            cos, sin = _rope_tables(rope, T, D, self.device, tiled)
            _lib.call("wf_fp8_kv_pack_rope_tiled", kp, vp, T, H, D, ld, cos.data_ptr(), sin.data_ptr(), cos.shape[0],
                      *pool_args)
            return
        _lib.call("wf_fp8_kv_pack", kp, vp, T, H, D, ld, *pool_args)

    def pack_k_norm_rope(self, k: torch.Tensor, v: torch.Tensor | None, table: PageTable, norm_w: torch.Tensor,
                         eps: float, rope: tuple[torch.Tensor, torch.Tensor] | None,
                         ku_out: torch.Tensor | None = None, q: torch.Tensor | None = None,
                         norm_q: torch.Tensor | None = None) -> None:
        """K straight from the QKV projection into the pages.

        k, v: [T, dim] bf16 rows (dim = H*D, token stride a multiple of 8, e.g.
        column views of a fused QKV output).  K gets WanRMSNorm over the row
        (norm_w [dim]), is written un-rotated to ``ku_out`` ([T, dim] bf16, may
        be ``k`` itself) if given, is rotated by ``rope = (cos, sin)`` and is
        packed; V is packed as by :meth:`pack`.  Equal, bit for bit, to
        wf_rmsnorm_rope followed by wf_fp8_kv_pack.  With ``q`` (and its
        RMSNorm weight ``norm_q``), Q's RMSNorm + RoPE runs in the same pass,
        in place (wf_qk_norm_rope_kv_pack).
        """
        for name, t in (("k", k), ("v", v), ("ku_out", ku_out), ("q", q)):
            if t is None:
                continue
            if t.dim() != 2 or t.dtype != torch.bfloat16 or t.stride(1) != 1:
                raise ValueError(f"{name} must be bf16 [T, dim] rows with unit column stride")
        T, dim = k.shape
        H, D = self.n_heads, self.head_dim
        if dim != H * D:
            raise ValueError(f"k rows have {dim} values; the pool holds {H} heads x {D}")
        if v is not None and (tuple(v.shape) != (T, dim) or (T > 1 and v.stride(0) != k.stride(0))):
            raise ValueError("v must match k's shape and token stride")
        if ku_out is not None and tuple(ku_out.shape) != (T, dim):
            raise ValueError("ku_out must be [T, dim]")
        if q is not None and (tuple(q.shape) != (T, dim) or norm_q is None):
            raise ValueError("q must be [T, dim] and comes with norm_q")
        if len(table) * self.page_tokens < T:
            raise RuntimeError(f"page table of {len(table)} pages cannot hold {T} tokens")
        cos = sin = None
        if rope is not None:
            cos, sin = _rope_tables(rope, T, D, self.device)
        ld = k.stride(0) if T > 1 else dim
        qargs = () if q is None else (q.data_ptr(), q.stride(0) if T > 1 else dim, norm_q.data_ptr())
        _lib.call(
            "wf_k_norm_rope_kv_pack" if q is None else "wf_qk_norm_rope_kv_pack", *qargs,
            k.data_ptr(), _lib.ptr(v), T, H, D, ld, float(eps), norm_w.data_ptr(), _lib.ptr(cos), _lib.ptr(sin),
            _lib.ptr(ku_out), (ku_out.stride(0) if T > 1 else dim) if ku_out is not None else 0,
            table.dev.data_ptr(), len(table), self.page_tokens,
            self.k_codes.data_ptr(), self.v_codes.data_ptr() if v is not None else None,
            self.k_scales.data_ptr(), self.v_scales.data_ptr() if v is not None else None,
            self.pool_pages,
            _lib.stream_handle(self.device),
        )

    def unpack(
        self,
        table: PageTable,
        n_tokens: int,
        with_v: bool = True,
        out_k: torch.Tensor | None = None,
        out_v: torch.Tensor | None = None,
    ):
        """Gather + dequantize ``n_tokens`` logical tokens to bf16 [T, H, D]."""
        if len(table) * self.page_tokens < n_tokens:
            raise RuntimeError(f"page table of {len(table)} pages cannot hold {n_tokens} tokens")
        shape = (n_tokens, self.n_heads, self.head_dim)
        if out_k is None:
            out_k = torch.empty(shape, dtype=torch.bfloat16, device=self.device)
        if with_v and out_v is None:
            out_v = torch.empty(shape, dtype=torch.bfloat16, device=self.device)
        for name, t in (("out_k", out_k), ("out_v", out_v if with_v else None)):
            if t is not None and (tuple(t.shape) != shape or t.dtype != torch.bfloat16 or not t.is_contiguous()):
                raise ValueError(f"{name} must be contiguous bf16 {shape}")
        _lib.call(
            "wf_fp8_kv_unpack",
            self.k_codes.data_ptr(), self.v_codes.data_ptr() if with_v else None,
            self.k_scales.data_ptr(), self.v_scales.data_ptr() if with_v else None,
            self.pool_pages, table.dev.data_ptr(), len(table), self.page_tokens,
            n_tokens, self.n_heads, self.head_dim,
            out_k.data_ptr(), out_v.data_ptr() if with_v else None,
            _lib.stream_handle(self.device),
        )
        return (out_k, out_v) if with_v else out_k


@dataclass
class PagedKV:
    """Page descriptor handed to the attention backend in place of dense K/V.

    ``n_tokens`` logical keys live in ``pool`` at the pages of ``table``.
    """

    pool: Fp8PagePool
    table: PageTable
    n_tokens: int

    @property
    def shape(self):
        # The reference reads ctx_k.shape[1] for its profile line (backend.py:151).
        return (1, self.n_tokens, self.pool.n_heads, self.pool.head_dim)


def fp8_encode(x: torch.Tensor) -> torch.Tensor:
    """e4m3fn codes (uint8) of an fp32 device tensor: torch's ``x.to(float8_e4m3fn)``."""
    if x.dtype != torch.float32:
        raise ValueError("fp8_encode expects float32")
    x = x.contiguous()
    out = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    _lib.call("wf_fp8_e4m3_encode_f32", x.data_ptr(), out.data_ptr(), x.numel(), _lib.stream_handle(x.device))
    return out


def fp8_decode(codes: torch.Tensor) -> torch.Tensor:
    """fp32 values of e4m3fn codes (uint8 device tensor)."""
    if codes.dtype != torch.uint8:
        raise ValueError("fp8_decode expects uint8 codes")
    codes = codes.contiguous()
    out = torch.empty(codes.shape, dtype=torch.float32, device=codes.device)
    _lib.call("wf_fp8_e4m3_decode_f32", codes.data_ptr(), out.data_ptr(), codes.numel(),
              _lib.stream_handle(codes.device))
    return out


def pack_pertensor(kv: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """The reference's per-tensor FP8 KV quantization (``_all_gather_fp8``,
    wave_rt/denoiser/exchange/common.py:145-150): bf16 K/V [..., D] ->
    (e4m3fn codes as uint8, same shape; fp32 scale [1]).  The scale is
    ``(amax|kv| / 448).clamp(min=1e-8)`` in bf16 arithmetic, then fp32; the
    quotient kv / scale is rounded to bf16 before the e4m3 cast."""
    if kv.dtype != torch.bfloat16:
        raise ValueError(f"pack_pertensor expects bf16 K/V, got {kv.dtype}")
    if kv.numel() == 0 or kv.shape[-1] % 8:
        raise ValueError(f"pack_pertensor needs a non-empty tensor whose last dim is a multiple of 8, got "
                         f"{tuple(kv.shape)}")
    kv = kv.contiguous()
    D = kv.shape[-1]
    codes = torch.empty(kv.shape, dtype=torch.uint8, device=kv.device)
    scale = torch.empty((1,), dtype=torch.float32, device=kv.device)
    partials = torch.empty((_lib.FP8_AMAX_PARTIALS,), dtype=torch.float32, device=kv.device)
    _lib.call("wf_fp8_quant_pertensor", kv.data_ptr(), kv.numel() // D, D, D, _lib.FP8_TENSOR_ACT, codes.data_ptr(),
              scale.data_ptr(), partials.data_ptr(), _lib.stream_handle(kv.device))
    return codes, scale


def unpack_pertensor(codes: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """fp32 ``codes.view(e4m3).to(bf16) * scale`` (common.py:161-164; the 1-element fp32 scale makes the
    result fp32)."""
    if codes.dtype != torch.uint8 or scale.dtype != torch.float32 or scale.numel() != 1:
        raise ValueError("unpack_pertensor takes uint8 codes and a 1-element fp32 scale")
    codes = codes.contiguous()
    out = torch.empty(codes.shape, dtype=torch.float32, device=codes.device)
    _lib.call("wf_fp8_dequant_pertensor_f32", codes.data_ptr(), scale.data_ptr(), codes.numel(), out.data_ptr(),
              _lib.stream_handle(codes.device))
    return out


def all_gather_fp8(mine: torch.Tensor, world: int = 1) -> list[torch.Tensor]:
    """``_all_gather_fp8`` (common.py:143-164) on one GPU: quantize this rank's K/V [2, T, H, D] per tensor and
    return the dequantized fp32 tensors of the ``world`` ranks, here all this rank's (a single-GPU gather of
    one rank's codes and scale is the identity)."""
    if world != 1:
        raise ValueError("one GPU holds one rank: world must be 1 (the multi-GPU gather is not built)")
    codes, scale = pack_pertensor(mine)
    return [unpack_pertensor(codes, scale)]
