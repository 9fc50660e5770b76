"""The allocation-free attention entry point (splat_kernel_attention_noalloc) against the
allocating one (splat_kernel_attention): same kernels and key-slice plan, the partials in the
library's static per-GPU scratch instead of the context's workspace. Two calls in a row, the
second smaller, each checked bit for bit against the allocating entry point on the same
inputs (and the first against an fp64 softmax(q k^T / 8) v), in bf16, f16 and fp32; a launch
whose partials exceed the scratch runs as one key slice (checked against fp64 on sampled
queries); two contexts calling it back to back without a synchronisation both get the
allocating entry point's result (the library orders the calls); and a call on a fresh context
leaves the device's free memory unchanged."""
import numpy as np
import pytest

from conftest import report

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _qkv(S, L, heads, tdt, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(S * L, 3 * heads * 64, generator=g) * 1.5).to(tdt)


def _fp64(qkv, S, L, heads, rows=None):
    """softmax(q k^T / 8) v in fp64, for every query or only the query rows `rows` (S == 1)."""
    x = qkv.double().reshape(S, L, 3, heads, 64).permute(2, 0, 3, 1, 4)
    q = x[0] if rows is None else x[0][:, :, rows]
    p = torch.softmax(q @ x[1].transpose(-1, -2) / 8.0, -1)
    n = L if rows is None else len(rows)
    return (p @ x[2]).permute(0, 2, 1, 3).reshape(S * n, heads * 64)


def _codes():
    import splathip
    return {"bf16": (splathip.BF16, torch.bfloat16), "f16": (splathip.F16, torch.float16),
            "f32": (splathip.F32, torch.float32)}


# (dtype, S, L, heads): key-sliced (the MapAnything C4 global block, 3 slices and 59 MB of
# partials; then 4500 tokens x 4 heads, 3 slices and 14 MB), the same in f16, then fp32 with slices
CASES = [("bf16", 1, 6223, 12), ("bf16", 1, 4500, 4), ("f16", 1, 6223, 12), ("f16", 1, 4500, 4),
         ("f32", 1, 700, 2)]


def test_noalloc_attention_matches_the_allocating_entry_point(ctx):
    for i, (dt, S, L, heads) in enumerate(CASES):
        report("noalloc.attention", call=i, dtype=dt, S=S, L=L, heads=heads)
        code, tdt = _codes()[dt]
        qkv = _qkv(S, L, heads, tdt, seed=100 + i).cuda()
        a = torch.full((S * L, heads * 64), float("nan"), dtype=tdt, device="cuda")
        b = torch.full((S * L, heads * 64), float("nan"), dtype=tdt, device="cuda")
        torch.cuda.synchronize()
        ctx.kernel_attention_noalloc(code, qkv.data_ptr(), a.data_ptr(), S, L, heads)
        ctx.kernel_attention(code, qkv.data_ptr(), b.data_ptr(), S, L, heads)
        ctx.synchronize()
        assert torch.equal(a.cpu(), b.cpu()), i
        if i in (0, 2):
            ref = _fp64(qkv.cpu(), S, L, heads)
            err = (a.cpu().double() - ref).abs().max().item() / ref.abs().max().item()
            report("noalloc.attention.err", dtype=dt, err=f"{err:.2e}")
            assert err < 2e-2


def test_noalloc_attention_beyond_its_scratch_runs_one_key_slice(ctx):
    """The C5 global block (24889 tokens x 12 heads: 236 MB of partials in 3 slices) runs unsplit
    in the allocation-free entry point; 96 sampled queries of every head against fp64."""
    S, L, heads = 1, 24889, 12
    report("noalloc.attention.unsplit", S=S, L=L, heads=heads)
    qkv = _qkv(S, L, heads, torch.bfloat16, seed=7).cuda()
    a = torch.full((L, heads * 64), float("nan"), dtype=torch.bfloat16, device="cuda")
    torch.cuda.synchronize()
    ctx.kernel_attention_noalloc(_codes()["bf16"][0], qkv.data_ptr(), a.data_ptr(), S, L, heads)
    ctx.synchronize()
    rows = torch.from_numpy(np.random.default_rng(3).choice(L, 96, replace=False))
    ref = _fp64(qkv.cpu(), S, L, heads, rows)
    got = a.cpu().double()[rows]
    err = (got - ref).abs().max().item() / ref.abs().max().item()
    report("noalloc.attention.unsplit.err", err=f"{err:.2e}")
    assert torch.isfinite(a.float()).all() and err < 2e-2


def test_noalloc_attention_two_contexts_are_ordered(ctx):
    """Two contexts (two streams) call the entry point back to back with key-sliced launches and
    no synchronisation between them: without the library's ordering their partials would
    overwrite each other in the one scratch."""
    import splathip
    code, tdt = _codes()["bf16"]
    ctx2 = splathip.Context(0)
    try:
        shapes = [(1, 6223, 12), (1, 4500, 4)]
        qkvs = [_qkv(S, L, h, tdt, seed=200 + k).cuda() for k, (S, L, h) in enumerate(shapes)]
        outs = [torch.full((S * L, h * 64), float("nan"), dtype=tdt, device="cuda") for S, L, h in shapes]
        want = [torch.full((S * L, h * 64), float("nan"), dtype=tdt, device="cuda") for S, L, h in shapes]
        torch.cuda.synchronize()
        for rep in range(3):
            report("noalloc.attention.two_contexts", rep=rep)
            for c, (S, L, h), q, o in zip((ctx, ctx2), shapes, qkvs, outs):
                c.kernel_attention_noalloc(code, q.data_ptr(), o.data_ptr(), S, L, h)
            ctx.synchronize()
            ctx2.synchronize()
            for (S, L, h), q, w in zip(shapes, qkvs, want):
                ctx.kernel_attention(code, q.data_ptr(), w.data_ptr(), S, L, h)
            ctx.synchronize()
            for k in range(2):
                assert torch.equal(outs[k].cpu(), want[k].cpu()), (rep, k)
    finally:
        ctx2.close()


def test_noalloc_attention_allocates_nothing(ctx):
    """A key-sliced call (59 MB of partials) on a fresh context, whose workspace was never sized,
    leaves the device's free memory as it was. The HIP runtime attaches a hardware queue (8 MiB)
    at a stream's first launch, so the fresh context first runs a small unsliced call."""
    import splathip
    code, tdt = _codes()["bf16"]
    S, L, heads = 1, 6223, 12
    qkv = _qkv(S, L, heads, tdt, seed=9).cuda()
    out = torch.empty((S * L, heads * 64), dtype=tdt, device="cuda")
    ctx.kernel_attention_noalloc(code, qkv.data_ptr(), out.data_ptr(), S, L, heads)  # code objects loaded
    ctx.synchronize()
    fresh = splathip.Context(0)
    try:
        fresh.kernel_attention_noalloc(code, qkv.data_ptr(), out.data_ptr(), 1, 64, 1)  # its stream's first launch
        fresh.synchronize()
        torch.cuda.synchronize()
        free0, _ = torch.cuda.mem_get_info()
        fresh.kernel_attention_noalloc(code, qkv.data_ptr(), out.data_ptr(), S, L, heads)
        fresh.synchronize()
        free1, _ = torch.cuda.mem_get_info()
    finally:
        fresh.close()
    report("noalloc.attention.free_memory", before=free0, after=free1)
    assert free1 == free0
