"""Size-independent properties of the paged FP8 attention, checked bit for bit at the full 1.3B size.

The oracle comparisons hold sampled query rows at 37440 keys (the CPU cannot attend all 4680 x 12 rows over
that context in seconds).  These tests cover every row of the full workload (4680 queries, 12 heads, 8 chunks
of 4680 keys in 1560-token pages, Q, K, V ~ N(0, 1)) without the oracle, through properties that any correct
kernel has and a plausible indexing mistake breaks:

* page placement is invisible: the same logical context packed into other physical pages (another pool
  size, another permutation of page ids) gives the same output bits, for the exact, quantized-QK and fp8-PV
  forms (a wrong page base, or scales read from the wrong page, changes them);
* the paged kernel over FP8 pages equals the dense kernel over the same pages unpacked to bf16 (the pages'
  gather-dequant values bf16(code * s), which the unpack kernel produces bit-exactly against the oracle):
  the decode inside the attention kernel is exactly the unpack's;
* query rows and heads are independent: a slice of query rows starting off any tile boundary, and one head
  packed alone into a one-head pool, reproduce the full call's rows and head bit for bit; with keys that grow
  from tile to tile and queries of mixed magnitude, so that some queries of a wave rescale and others do not,
  rows in another order or alone still reproduce theirs (each query keeps its own running maximum).
"""

import pytest
import torch

from waveforcing_amd import inputs
from waveforcing_amd.backend import attn_dense_bf16, attn_paged_fp8
from waveforcing_amd.kv import Fp8PagePool, PagedKV

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
LQ, H, D, PAGE, CHUNKS = 4680, 12, 128, 1560, 8
N_KV = CHUNKS * 4680
FORMS = {"exact": {}, "quantized_qk": {"quantized_qk": True}, "fp8_pv": {"fp8_pv": True}}


def _normal(shape, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return torch.randn(shape, generator=g, device=DEV).to(torch.bfloat16)


def _context(k, v, pool_pages, seed, heads=H, page=PAGE):
    n_pages = -(-k.shape[0] // page)
    pool = Fp8PagePool(pool_pages, heads, D, page, DEV)
    table = pool.page_table(inputs.page_table(n_pages, pool_pages, seed=seed))
    pool.pack(k, v, table)
    return PagedKV(pool, table, k.shape[0])


@pytest.fixture(scope="module")
def full():
    q = _normal((LQ, H, D), 900)
    k = _normal((N_KV, H, D), 901)
    v = _normal((N_KV, H, D), 902)
    ctx = _context(k, v, 2 * N_KV // PAGE, seed=903)
    outs = {name: attn_paged_fp8(q, ctx, **kw) for name, kw in FORMS.items()}
    torch.cuda.synchronize()
    return q, k, v, ctx, outs


@pytest.mark.parametrize("form", list(FORMS))
def test_page_placement_is_invisible(full, form):
    q, k, v, _, outs = full
    other = _context(k, v, N_KV // PAGE + 5, seed=904)
    assert other.table.host != full[3].table.host
    out = attn_paged_fp8(q, other, **FORMS[form])
    assert torch.equal(out, outs[form])


def test_paged_equals_dense_over_unpacked_pages(full):
    q, _, _, ctx, outs = full
    kb, vb = ctx.pool.unpack(ctx.table, N_KV)
    assert torch.equal(attn_dense_bf16(q, kb, vb), outs["exact"])


@pytest.mark.parametrize("n_kv", [1, 63, 64, 1561, 3 * PAGE + 77])
def test_paged_equals_dense_over_unpacked_pages_ragged(n_kv):
    """Contexts that end inside a tile or a page, with a 300-query tail tile and 3 heads."""
    q = _normal((300, 3, D), 910 + n_kv)
    k, v = _normal((n_kv, 3, D), 920 + n_kv), _normal((n_kv, 3, D), 930 + n_kv)
    ctx = _context(k, v, -(-n_kv // PAGE) + 2, seed=940 + n_kv, heads=3)
    kb, vb = ctx.pool.unpack(ctx.table, n_kv)
    assert torch.equal(attn_dense_bf16(q, kb, vb), attn_paged_fp8(q, ctx))


@pytest.mark.parametrize("form", list(FORMS))
def test_query_rows_are_independent(full, form):
    q, _, _, ctx, outs = full
    a, b = 1000, 1333  # off the 32-row wave and 256-row workgroup boundaries
    out = attn_paged_fp8(q[a:b], ctx, **FORMS[form])
    assert torch.equal(out, outs[form][a:b])


@pytest.mark.parametrize("form", list(FORMS))
def test_one_head_alone_equals_its_head_of_the_full_call(full, form):
    q, k, v, _, outs = full
    h = 7
    one = _context(k[:, h:h + 1].contiguous(), v[:, h:h + 1].contiguous(), N_KV // PAGE + 3, seed=905, heads=1)
    out = attn_paged_fp8(q[:, h:h + 1].contiguous(), one, **FORMS[form])
    assert torch.equal(out[:, 0], outs[form][:, h])


@pytest.mark.parametrize("form", list(FORMS))
def test_rows_are_independent_when_some_queries_rescale(form):
    """Keys from the eleventh 64-key tile on are 4x larger and the first half of the queries is scaled down
    64x: a large query's scores there exceed its running maximum by more than the rescale threshold (2^8 in
    the weights), a small query's never do (its softmax stays nearly flat, so a moved maximum would show in
    the rounding of its weights).  In the full call the small queries fill waves of their own; in a shuffled
    order they share waves with large ones.  Rows computed in that order, or as a slice across a wave of each
    kind, still equal their rows of the full call bit for bit."""
    Lq, h, n_kv, page = 600, 2, 64 * 20 + 9, 200
    q = _normal((Lq, h, D), 960)
    q = q * torch.where(torch.arange(Lq, device=DEV) < Lq // 2, 1.0 / 64, 1.0)[:, None, None].to(torch.bfloat16)
    grow = torch.where(torch.arange(n_kv, device=DEV) >= 640, 4.0, 1.0)[:, None, None]
    k = (_normal((n_kv, h, D), 961).float() * grow).to(torch.bfloat16)
    v = _normal((n_kv, h, D), 962)
    ctx = _context(k, v, -(-n_kv // page) + 3, seed=963, heads=h, page=page)
    full = attn_paged_fp8(q, ctx, **FORMS[form])
    perm = torch.randperm(Lq, generator=torch.Generator().manual_seed(964)).to(DEV)
    assert torch.equal(attn_paged_fp8(q[perm].contiguous(), ctx, **FORMS[form]), full[perm])
    assert torch.equal(attn_paged_fp8(q[270:351], ctx, **FORMS[form]), full[270:351])
