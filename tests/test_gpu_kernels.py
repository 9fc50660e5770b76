"""Kernel-level parity of the MFMA GEMM and the flash-attention kernel (through the C ABI's
kernel entry points, include/splathip_kernels.h) against plain PyTorch fp32/fp64 references
of the same op on the same bf16/fp32-rounded operands."""
import numpy as np
import pytest

from conftest import report

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _dt(name):
    import splathip
    return (splathip.BF16, torch.bfloat16) if name == "bf16" else (splathip.F32, torch.float32)


GEMM_CASES = [
    # (M, N, K, act)
    (1, 64, 64, 0),
    (100, 100, 64, 1),
    (333, 32, 288, 0),
    (777, 64, 576, 2),
    (1297, 1152, 384, 0),
    (5838, 384, 1536, 0),
    (129, 130, 784, 1),
    (2500, 3072, 1024, 2),
]


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("M,N,K,act", GEMM_CASES)
def test_gemm_matches_torch(ctx, dtype, M, N, K, act):
    report("gemm", dtype=dtype, M=M, N=N, K=K, act=act)
    code, tdt = _dt(dtype)
    g = torch.Generator().manual_seed(M * 7 + N * 3 + K)
    A = torch.randn(M, K, generator=g).to(tdt)
    ldw = (K + 63) // 64 * 64
    Wm = torch.zeros(N, ldw)
    Wm[:, :K] = torch.randn(N, K, generator=g) * 0.05
    Wm = Wm.to(tdt)
    bias = torch.randn(N, generator=g)
    dA, dW, db = A.cuda(), Wm.cuda(), bias.cuda()
    out = torch.empty(M, N, dtype=torch.float32, device="cuda")
    ctx.kernel_gemm(code, dA.data_ptr(), M, K, dW.data_ptr(), N, ldw, db.data_ptr(), act, out.data_ptr(), True)
    ctx.synchronize()
    ref = A.double() @ Wm[:, :K].double().T + bias.double()
    if act == 1:
        ref = torch.relu(ref)
    elif act == 2:
        ref = torch.nn.functional.gelu(ref)
    got = out.cpu().double()
    err = (got - ref).abs().max().item() / (ref.abs().max().item() + 1e-12)
    report("gemm.err", err=f"{err:.2e}")
    assert err < (1e-5 if dtype == "f32" else 2e-5), err
    # bf16/fp32 output storage path
    out2 = torch.empty(M, N, dtype=tdt, device="cuda")
    ctx.kernel_gemm(code, dA.data_ptr(), M, K, dW.data_ptr(), N, ldw, db.data_ptr(), act, out2.data_ptr(), False)
    ctx.synchronize()
    err2 = (out2.cpu().double() - ref).abs().max().item() / (ref.abs().max().item() + 1e-12)
    assert err2 < (1e-5 if dtype == "f32" else 8e-3), err2


ATTN_CASES = [
    # (S, L, heads)
    (1, 1, 1),
    (1, 65, 2),
    (3, 130, 1),
    (6, 973, 6),
    (1, 5838, 6),
    (2, 1037, 16),
]


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("S,L,heads", ATTN_CASES)
def test_attention_matches_torch(ctx, dtype, S, L, heads):
    if dtype == "f32" and S * L > 6000:
        pytest.skip("fp32 covered at smaller sizes")
    report("attention", dtype=dtype, S=S, L=L, heads=heads)
    code, tdt = _dt(dtype)
    g = torch.Generator().manual_seed(S * 1000 + L + heads)
    qkv = (torch.randn(S * L, 3 * heads * 64, generator=g) * 1.5).to(tdt)
    dq = qkv.cuda()
    out = torch.empty(S * L, heads * 64, dtype=tdt, device="cuda")
    ctx.kernel_attention(code, dq.data_ptr(), out.data_ptr(), S, L, heads)
    ctx.synchronize()
    x = dq.double().reshape(S, L, 3, heads, 64).permute(2, 0, 3, 1, 4)  # [3, S, h, L, 64]
    q, k, v = x[0], x[1], x[2]
    p = torch.softmax(q @ k.transpose(-1, -2) / 8.0, -1)
    ref = (p @ v).permute(0, 2, 1, 3).reshape(S * L, heads * 64).cpu()
    got = out.cpu().double()
    err = (got - ref).abs().max().item() / (ref.abs().max().item() + 1e-12)
    report("attention.err", err=f"{err:.2e}")
    assert err < (2e-5 if dtype == "f32" else 2e-2), err
