"""The allocation-free attention entry point (splat_kernel_attention_noalloc) against the
allocating one (splat_kernel_attention): same kernels and key-slice plan, the partials in the
library's static per-GPU scratch instead of the context's workspace. Two calls in a row, the
second smaller, each checked bit for bit against the allocating entry point on the same
inputs (and the first against an fp64 softmax(q k^T / 8) v); a launch whose partials exceed
the scratch is refused before anything runs."""
import numpy as np
import pytest

from conftest import report

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _qkv(S, L, heads, tdt, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(S * L, 3 * heads * 64, generator=g) * 1.5).to(tdt)


def _fp64(qkv, S, L, heads):
    x = qkv.double().reshape(S, L, 3, heads, 64).permute(2, 0, 3, 1, 4)
    p = torch.softmax(x[0] @ x[1].transpose(-1, -2) / 8.0, -1)
    return (p @ x[2]).permute(0, 2, 1, 3).reshape(S * L, heads * 64)


# (S, L, heads): both key-sliced (the MapAnything C4 global block, 3 slices and 59 MB of
# partials; then 4500 tokens x 4 heads, 3 slices and 14 MB), then fp32 with slices
CASES = [("bf16", 1, 6223, 12), ("bf16", 1, 4500, 4), ("f32", 1, 700, 2)]


def test_noalloc_attention_matches_the_allocating_entry_point(ctx):
    import splathip
    for i, (dt, S, L, heads) in enumerate(CASES):
        report("noalloc.attention", call=i, dtype=dt, S=S, L=L, heads=heads)
        code, tdt = (splathip.BF16, torch.bfloat16) if dt == "bf16" else (splathip.F32, torch.float32)
        qkv = _qkv(S, L, heads, tdt, seed=100 + i).cuda()
        a = torch.full((S * L, heads * 64), float("nan"), dtype=tdt, device="cuda")
        b = torch.full((S * L, heads * 64), float("nan"), dtype=tdt, device="cuda")
        torch.cuda.synchronize()
        ctx.kernel_attention_noalloc(code, qkv.data_ptr(), a.data_ptr(), S, L, heads)
        ctx.kernel_attention(code, qkv.data_ptr(), b.data_ptr(), S, L, heads)
        ctx.synchronize()
        assert torch.equal(a.cpu(), b.cpu()), i
        if i == 0:
            ref = _fp64(qkv.cpu(), S, L, heads)
            err = (a.cpu().double() - ref).abs().max().item() / ref.abs().max().item()
            report("noalloc.attention.err", err=f"{err:.2e}")
            assert err < 2e-2


def test_noalloc_attention_refuses_partials_beyond_its_scratch(ctx):
    import splathip
    S, L, heads = 1, 24889, 12   # the C5 global block: 3 key slices, 236 MB of partials
    with pytest.raises(splathip.SplatError) as e:
        ctx.kernel_attention_noalloc(splathip.BF16, 0, 0, S, L, heads)
    assert e.value.code == splathip.BAD_ARGUMENT and "scratch" in str(e.value)
