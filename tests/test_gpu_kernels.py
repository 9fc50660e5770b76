"""Kernel-level parity of the MFMA GEMM and the flash-attention kernel (through the C ABI's
kernel entry points, include/splathip_kernels.h) against plain PyTorch fp32/fp64 references
of the same op on the same bf16/f16/fp32-rounded operands.

Bounds on a result stored in a 16-bit type are set by its rounding: half an ulp is 2^-9 of the
value in bf16 (8 mantissa bits) and 2^-12 in f16 (11 bits), so the f16 bounds sit 4-8x below
the bf16 ones."""
import math

import numpy as np
import pytest

from conftest import report

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _dt(name):
    import splathip
    return {"bf16": (splathip.BF16, torch.bfloat16), "f16": (splathip.F16, torch.float16),
            "f32": (splathip.F32, torch.float32)}[name]


def _tol(dtype, f32, bf16, f16):
    return {"f32": f32, "bf16": bf16, "f16": f16}[dtype]


DTYPES = ["bf16", "f16", "f32"]


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
    (6000, 3072, 1024, 2),  # 320x256 tiles (228: one round of 256 CUs)
    (6000, 1536, 512, 1),   # 320x128 tiles (228)
    (6000, 768, 768, 0),    # 192x128 tiles (192)
    # 400 tiles of 256x256: a second round of 144 tiles (the MapAnything encoder's fc1 shape)
    (6222, 4096, 1024, 2),
    # split-K (fewer tiles than half a round of CUs, K >= 16 k-tiles): fp32 partials + reduce
    (100, 256, 4096, 0),
    (777, 64, 2048, 2),
    (300, 1001, 2048, 1),
    # DA3-Small C1 shapes (1297 rows, K = 384): few tiles, K too short to split
    (1297, 384, 384, 0),
    (1297, 1536, 384, 2),
]


@pytest.mark.parametrize("dtype", DTYPES)
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
    torch.cuda.synchronize()  # inputs were written on torch's stream, the library runs on its own
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
    # output stored in the operands' type
    out2 = torch.empty(M, N, dtype=tdt, device="cuda")
    torch.cuda.synchronize()  # inputs were written on torch's stream, the library runs on its own
    ctx.kernel_gemm(code, dA.data_ptr(), M, K, dW.data_ptr(), N, ldw, db.data_ptr(), act, out2.data_ptr(), False)
    ctx.synchronize()
    err2 = (out2.cpu().double() - ref).abs().max().item() / (ref.abs().max().item() + 1e-12)
    assert err2 < _tol(dtype, 1e-5, 8e-3, 1e-3), err2


@pytest.mark.parametrize("dtype", DTYPES)
def test_gemm_gelu_epilogue_accuracy(ctx, dtype):
    """The epilogue's GELU against the exact erf GELU over [-9, 9]: out[m, n] = x_m (A's first
    column, W's first row of ones), so the GEMM adds no rounding and the check is the
    activation's own error, <= 3e-7 * max(1, |x|) (erfc approximation error 1.5e-7, plus fp32
    rounding)."""
    code, tdt = _dt(dtype)
    M, N, K = 4096, 64, 64
    x = torch.linspace(-9, 9, M).to(tdt).double()
    A = torch.zeros(M, K, dtype=tdt)
    A[:, 0] = x.to(tdt)
    Wm = torch.zeros(N, K, dtype=tdt)
    Wm[:, 0] = 1
    bias = torch.zeros(N)
    dA, dW, db = A.cuda(), Wm.cuda(), bias.cuda()
    out = torch.empty(M, N, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    ctx.kernel_gemm(code, dA.data_ptr(), M, K, dW.data_ptr(), N, K, db.data_ptr(), 2, out.data_ptr(), True)
    ctx.synchronize()
    ref = torch.nn.functional.gelu(x)[:, None].expand(M, N)
    err = ((out.cpu().double() - ref).abs() / x.abs().clamp(min=1)[:, None]).max().item()
    report("gemm.gelu", dtype=dtype, err=f"{err:.2e}")
    assert err <= 3e-7, err


ATTN_CASES = [
    # (S, L, heads)
    (1, 1, 1),
    (1, 65, 2),
    (3, 130, 1),
    (6, 973, 6),
    (1, 1297, 6),    # DA3-Small C1 (fp32: 7 key slices of 32-key tiles)
    (1, 5838, 6),    # DA3-Small C2 global: 138 blocks of 256 queries in 3 key slices, ragged last tile
    (2, 1037, 16),
    (6, 1037, 16),   # the C4 encoder's per-view shape: 480 blocks of 256 queries, two query sub-tiles per wave
    (6, 1100, 16),   # the same with another ragged last key tile
    (7, 1037, 16),   # 1008 blocks of 128 queries: one query sub-tile per wave, ragged last key tile
    (9, 1100, 12),   # 972 blocks: the same with another ragged end
    # long sequences: key slices merged by a second kernel where the grid leaves block slots idle
    (1, 6223, 12),   # the MapAnything C4 global block (588 blocks: 512 whole, the 76 left in 3 key slices)
    (1, 4096, 33),   # two query sub-tiles per wave, 528 blocks: 512 whole, 16 in 4 slices, no ragged tile
    # tail splits: two sequences (576 blocks: 512 whole, 64 in 4 slices), and 561 blocks
    (2, 4500, 8),
    (1, 4100, 17),
    # two query sub-tiles per wave: 544 blocks, 512 whole and 32 in 4 slices, ragged last key tile
    (2, 4100, 16),
]


@pytest.mark.parametrize("dtype", DTYPES)
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
    torch.cuda.synchronize()  # inputs were written on torch's stream, the library runs on its own
    ctx.kernel_attention(code, dq.data_ptr(), out.data_ptr(), S, L, heads)
    ctx.synchronize()
    x = dq.double().reshape(S, L, 3, heads, 64).permute(2, 0, 3, 1, 4)  # [3, S, h, L, 64]
    q, k, v = x[0], x[1], x[2]
    p = torch.softmax(q @ k.transpose(-1, -2) / 8.0, -1)
    ref = (p @ v).permute(0, 2, 1, 3).reshape(S * L, heads * 64).cpu()
    got = out.cpu().double()
    err = (got - ref).abs().max().item() / (ref.abs().max().item() + 1e-12)
    report("attention.err", err=f"{err:.2e}")
    assert err < _tol(dtype, 2e-5, 2e-2, 4e-3), err


# The 16-bit kernels' softmax scale: Q times log2(e)/8 in fp32, rounded to bf16 or f16 (a second
# rounding of Q when, as through splat_kernel_attention, Q arrives unscaled), then weights
# 2^(q'.k).
Q_SCALE = float(np.float32(0.125) * np.float32(1.4426950408889634))


def _attention_ref_scaled(dq, S, L, heads):
    x = dq.float().reshape(S, L, 3, heads, 64).permute(2, 0, 3, 1, 4)  # [3, S, h, L, 64]
    q = x[0] * np.float32(Q_SCALE)  # fp32: the kernel scales Q in fp32 and keeps it there
    q = (q.to(dq.dtype) if dq.dtype != torch.float32 else q).double()
    p = torch.softmax((q @ x[1].double().transpose(-1, -2)) * math.log(2.0), -1)
    return (p @ x[2].double()).permute(0, 2, 1, 3).reshape(S * L, heads * 64).cpu()


# Logits far outside the usual range, which move the kernel's per-query exponent reference off
# zero (sums of 2^s beyond 2^64 or below 2^-64): all keys far above, all far below, one key far
# above the rest in a late tile, and a mix of queries in each regime. Shapes: one and two query
# sub-tiles per wave, with and without key slices, ragged last tiles. At logits of hundreds the
# rounding of Q alone moves them by units, so the reference follows the kernel's Q rounding and
# the test checks the softmax and its reference moves, at the usual tolerance. In f16 the kernel
# keeps the running reference from the first tile (weights at most 2^8, inside f16's range);
# "high" is the case whose weights 2^s would pass f16's 65504 without it.
EXTREME_CASES = ["high", "low", "late_peak", "mixed"]


@pytest.mark.parametrize("dtype,S,L,heads", [("bf16", 2, 1037, 3), ("bf16", 7, 1037, 16), ("bf16", 1, 6223, 2),
                                             ("bf16", 2, 4500, 8), ("bf16", 2, 4100, 16),
                                             ("f16", 2, 1037, 3), ("f16", 7, 1037, 16), ("f16", 1, 6223, 2),
                                             ("f32", 1, 1297, 6), ("f32", 3, 130, 2)])
@pytest.mark.parametrize("kind", EXTREME_CASES)
def test_attention_extreme_logits(ctx, kind, dtype, S, L, heads):
    report("attention.extreme", kind=kind, dtype=dtype, S=S, L=L, heads=heads)
    code, tdt = _dt(dtype)
    g = torch.Generator().manual_seed(L + heads + len(kind))
    x = torch.randn(S, L, 3, heads, 64, generator=g)
    u = torch.randn(S, 1, heads, 64, generator=g)
    u = u / u.norm(dim=-1, keepdim=True)
    if kind == "high":    # every logit about +600 (natural units), spread of a few units
        x[:, :, 1] = 8.0 * u + 0.3 * x[:, :, 1]
        x[:, :, 0] = 600.0 * u + 0.3 * x[:, :, 0]
    elif kind == "low":   # every logit about -400
        x[:, :, 1] = 8.0 * u + 0.3 * x[:, :, 1]
        x[:, :, 0] = -400.0 * u + 0.3 * x[:, :, 0]
    elif kind == "late_peak":  # ordinary logits, then one key per sequence at +300 in a late tile
        x[:, :, 0] = 8.0 * u + 0.5 * x[:, :, 0]
        x[:, L - 40, 1] = 300.0 * u[:, 0]
    else:                 # queries alternate between the three regimes
        x[:, :, 1] = 8.0 * u + 0.3 * x[:, :, 1]
        scale = torch.tensor([600.0, -400.0, 1.0]).repeat(L // 3 + 1)[:L].view(1, L, 1, 1)
        x[:, :, 0] = scale * u + 0.3 * x[:, :, 0]
    qkv = x.reshape(S * L, 3 * heads * 64).to(tdt)
    dq = qkv.cuda()
    out = torch.empty(S * L, heads * 64, dtype=tdt, device="cuda")
    torch.cuda.synchronize()
    ctx.kernel_attention(code, dq.data_ptr(), out.data_ptr(), S, L, heads)
    ctx.synchronize()
    ref = _attention_ref_scaled(dq, S, L, heads)
    got = out.cpu().double()
    assert torch.isfinite(got).all()
    err = (got - ref).abs().max().item() / (ref.abs().max().item() + 1e-12)
    report("attention.extreme.err", err=f"{err:.2e}")
    # fp32: at logits near +600 (865 in base 2) fp32 holds the exponent itself to ~5e-5, so the
    # weights carry ~1e-4 relative error whatever the kernel does
    assert err < _tol(dtype, 1e-3, 2e-2, 4e-3), err


CONV_CASES = [
    # (V, H, W, Cin, Cout, ks, stride, relu_in, act, residual)
    (1, 5, 7, 8, 8, 3, 1, 0, 0, False),
    (2, 16, 12, 48, 64, 3, 1, 0, 0, False),
    (2, 16, 12, 64, 64, 3, 1, 1, 1, True),
    (1, 27, 36, 384, 384, 3, 2, 0, 0, False),
    (3, 13, 9, 32, 7, 3, 1, 0, 1, False),
    (2, 10, 11, 96, 256, 1, 1, 0, 0, True),
    (1, 28, 37, 256, 128, 3, 1, 0, 0, False),
    # split-K: the DPT head's coarsest level (M = 1596, K = 6912) and a narrow conv
    (6, 19, 14, 768, 256, 3, 1, 0, 0, True),
    (2, 9, 7, 512, 64, 3, 1, 1, 1, False),
    # Cin a multiple of 32 but not 64: per-tap path on 32-element k-tiles (bf16), bias; ReLU-on-load
    # + residual; split-K (K = 1440)
    (2, 16, 12, 96, 64, 3, 1, 0, 0, False),
    (1, 28, 37, 96, 256, 3, 1, 1, 1, True),
    (1, 9, 7, 160, 64, 3, 1, 0, 0, False),
    # 128 output channels over >= 768 tiles of 192 rows: the two-blocks-per-CU tile (bf16),
    # bias + ReLU epilogue, then ReLU-on-load with a residual (the full epilogue)
    (3, 224, 224, 64, 128, 3, 1, 0, 1, False),
    (3, 224, 224, 64, 128, 3, 1, 1, 0, True),
    # Cin = 96 on the per-tap path with 32-element k-tiles (bf16) through the 256-row tiles:
    # 256x256 with three stages (the MapAnything level-0 layer_rn conv, 96 -> 256 at 112x148),
    # and 256x128 with ReLU-on-load and a residual
    (3, 112, 148, 96, 256, 3, 1, 0, 0, False),
    (3, 88, 94, 96, 256, 3, 1, 1, 1, True),
    # 389 tiles of 256x256 (the DPT heads' finest 256-channel maps, 6 x 112 x 148 pixels, 1.52
    # rounds): per-tap path with ReLU-on-load and a residual, then Cin = 96 (32-element k-tiles)
    # with bias + ReLU
    (6, 112, 148, 128, 256, 3, 1, 1, 0, True),
    (6, 112, 148, 96, 256, 3, 1, 0, 1, False),
    # Cin = 32 to at most 32 channels (the DA3 heads' full-resolution convs): the 128x32 tile on
    # the per-lane im2col path (no ReLU-on-load there); bias + ReLU, then a residual and 24 ragged
    # output channels
    (2, 40, 50, 32, 32, 3, 1, 0, 1, False),
    (3, 64, 80, 32, 24, 3, 1, 0, 0, True),
    # 3x3 stride 1 with Cin and Cout in {32, 64} and rows of at least 64 pixels (the DA3-Small
    # heads): the persistent halo kernel (16-bit types), tiles of 8 x 32 pixels with ragged last
    # rows and columns; ReLU-on-load + ReLU, a residual, every Cin / Cout pair, and 260 tiles
    # (blocks that take two)
    (2, 108, 144, 64, 64, 3, 1, 1, 1, False),
    (2, 108, 144, 64, 64, 3, 1, 0, 0, True),
    (3, 72, 96, 64, 32, 3, 1, 0, 0, False),
    (2, 70, 100, 32, 64, 3, 1, 0, 1, False),
    (1, 126, 168, 32, 32, 3, 1, 1, 1, True),
    (4, 100, 130, 64, 64, 3, 1, 1, 0, True),
]
H16_ONLY = {(3, 112, 148, 96, 256), (3, 88, 94, 96, 256), (6, 112, 148, 128, 256), (6, 112, 148, 96, 256)}


def bf16_tile(M, N, conv):
    """The 16-bit tile the library's picker (gemm.hip pick_bf16) chooses for an M x N launch:
    the fewest rounds of 256 CUs weighted by each tile's relative per-flop cost."""
    if conv == "halo":
        return "halo 8x32"
    if N <= 32:
        return "128x32"
    if N <= 64:
        return "128x64"
    if conv and N == 128 and -(-M // 192) >= 3 * 256:
        return "192x128 (2 per CU)"
    best, pick = None, None
    for (bm, bn), eff in (((256, 256), 1.0), ((256, 128), 0.8), ((320, 256), 1.0), ((320, 128), 0.8),
                          ((192, 128), 0.75), ((128, 128), 0.65)):
        tiles = -(-M // bm) * -(-N // bn)
        cost = -(-tiles // 256) * bm * bn / eff
        if best is None or cost < best * 0.999:
            best, pick = cost, f"{bm}x{bn}"
    return pick


def _conv_kind(ks, stride, Cin, Cout, Wo):
    """gemm.hip conv_halo_ok: which 16-bit convolutions take the halo kernel."""
    if ks == 3 and stride == 1 and Cin in (32, 64) and Cout in (32, 64) and Wo >= 64:
        return "halo"
    return ks > 1


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("V,H,W,Cin,Cout,ks,stride,relu_in,act,residual", CONV_CASES)
def test_conv2d_matches_torch(ctx, dtype, V, H, W, Cin, Cout, ks, stride, relu_in, act, residual):
    if dtype == "f32" and (V, H, W, Cin, Cout) in H16_ONLY:
        pytest.skip("a 16-bit tile-path case (fp32 picks its own tiles)")
    pad = ks // 2
    Ho, Wo = (H + 2 * pad - ks) // stride + 1, (W + 2 * pad - ks) // stride + 1
    report("conv2d", dtype=dtype, V=V, H=H, W=W, Cin=Cin, Cout=Cout, ks=ks, stride=stride,
           tile=bf16_tile(V * Ho * Wo, Cout, _conv_kind(ks, stride, Cin, Cout, Wo)) if dtype != "f32" else "fp32")
    code, tdt = _dt(dtype)
    F = torch.nn.functional
    g = torch.Generator().manual_seed(V * 31 + H * 7 + Cin + Cout)
    x = torch.randn(V, Cin, H, W, generator=g).to(tdt)
    w = (torch.randn(Cout, Cin, ks, ks, generator=g) * 0.05).to(tdt)
    b = torch.randn(Cout, generator=g)
    K = ks * ks * Cin
    ldw = (K + 63) // 64 * 64
    wp = torch.zeros(Cout, ldw, dtype=tdt)
    wp[:, :K] = w.permute(0, 2, 3, 1).reshape(Cout, K)
    xin = torch.relu(x.double()) if relu_in else x.double()
    ref = F.conv2d(xin, w.double(), b.double(), stride=stride, padding=pad)
    if act == 1:
        ref = torch.relu(ref)
    res = None
    if residual:
        res = torch.randn(V, Cout, Ho, Wo, generator=g).to(tdt)
        ref = ref + res.double()
    dx = x.permute(0, 2, 3, 1).contiguous().cuda()
    dres = res.permute(0, 2, 3, 1).contiguous().cuda() if residual else None
    out = torch.empty(V, Ho, Wo, Cout, dtype=tdt, device="cuda")
    dw, db = wp.cuda(), b.cuda()
    torch.cuda.synchronize()  # inputs were written on torch's stream, the library runs on its own
    ctx.kernel_conv2d(code, dx.data_ptr(), V, H, W, Cin, dw.data_ptr(), Cout, ldw, ks, stride, db.data_ptr(),
                      relu_in, act, dres.data_ptr() if residual else 0, out.data_ptr())
    ctx.synchronize()
    got = out.cpu().double().permute(0, 3, 1, 2)
    err = (got - ref).abs().max().item() / (ref.abs().max().item() + 1e-12)
    report("conv2d.err", err=f"{err:.2e}")
    assert err < _tol(dtype, 1e-5, 8e-3, 1e-3), err


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("V,R,Cc,Cin,Cout,s", [(1, 3, 4, 48, 48, 4), (2, 27, 36, 96, 96, 2), (2, 5, 3, 32, 16, 4)])
def test_conv_transpose2d_matches_torch(ctx, dtype, V, R, Cc, Cin, Cout, s):
    report("convT", dtype=dtype, V=V, R=R, C=Cc, Cin=Cin, Cout=Cout, s=s)
    code, tdt = _dt(dtype)
    g = torch.Generator().manual_seed(R * 100 + Cc + s)
    x = torch.randn(V, Cin, R, Cc, generator=g).to(tdt)
    w = (torch.randn(Cin, Cout, s, s, generator=g) * 0.05).to(tdt)
    b = torch.randn(Cout, generator=g)
    ref = torch.nn.functional.conv_transpose2d(x.double(), w.double(), b.double(), stride=s)
    ldw = (Cin + 63) // 64 * 64
    wp = torch.zeros(s * s * Cout, ldw, dtype=tdt)
    wp[:, :Cin] = w.permute(2, 3, 1, 0).reshape(s * s * Cout, Cin)
    bx = b.repeat(s * s)
    dx = x.permute(0, 2, 3, 1).contiguous().cuda()
    out = torch.empty(V, R * s, Cc * s, Cout, dtype=tdt, device="cuda")
    dw, db = wp.cuda(), bx.cuda()
    torch.cuda.synchronize()  # inputs were written on torch's stream, the library runs on its own
    ctx.kernel_conv_transpose2d(code, dx.data_ptr(), V, R, Cc, Cin, dw.data_ptr(), Cout, ldw, s, db.data_ptr(),
                                out.data_ptr())
    ctx.synchronize()
    got = out.cpu().double().permute(0, 3, 1, 2)
    err = (got - ref).abs().max().item() / (ref.abs().max().item() + 1e-12)
    assert err < _tol(dtype, 1e-5, 8e-3, 1e-3), err


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("V,Hi,Wi,C,Ho,Wo", [(1, 4, 3, 8, 8, 6), (2, 14, 18, 64, 27, 36), (1, 224, 296, 32, 392, 518),
                                              (1, 1, 5, 4, 3, 10), (2, 7, 7, 16, 7, 7)])
def test_resize_bilinear_matches_torch(ctx, dtype, V, Hi, Wi, C, Ho, Wo):
    report("resize", dtype=dtype, V=V, Hi=Hi, Wi=Wi, C=C, Ho=Ho, Wo=Wo)
    code, tdt = _dt(dtype)
    g = torch.Generator().manual_seed(Hi * 100 + Wi + Ho)
    x = torch.randn(V, C, Hi, Wi, generator=g).to(tdt)
    ref = torch.nn.functional.interpolate(x.double(), size=(Ho, Wo), mode="bilinear", align_corners=True)
    dx = x.permute(0, 2, 3, 1).contiguous().cuda()
    out = torch.empty(V, Ho, Wo, C, dtype=tdt, device="cuda")
    torch.cuda.synchronize()  # inputs were written on torch's stream, the library runs on its own
    ctx.kernel_resize_bilinear(code, dx.data_ptr(), V, Hi, Wi, C, out.data_ptr(), Ho, Wo)
    ctx.synchronize()
    got = out.cpu().double().permute(0, 3, 1, 2)
    err = (got - ref).abs().max().item() / (ref.abs().max().item() + 1e-12)
    assert err < _tol(dtype, 1e-6, 8e-3, 1e-3), err


# --- LayerNorm folded into the block GEMMs (GemmArgs::ln_in / ln_out) ----------------------

def _group_sums(x, group):
    """(sum, sum of squares) of fp32 rows per group of columns, fp64: [M, K/group, 2]."""
    M, K = x.shape
    g = x.double().reshape(M, K // group, group)
    return torch.stack([g.sum(-1), (g * g).sum(-1)], -1)


LN_CONSUMER_CASES = [
    # (M, N, K, act, group): qkv (act 0) and fc1 (act 2) shapes of the networks and the tiles they take
    (6222, 3072, 1024, 0, 64),   # MapAnything encoder qkv: 320x256 tiles
    (6222, 4096, 1024, 2, 64),   # encoder fc1 (GELU): 256x256
    (6223, 2304, 768, 0, 64),    # info-sharing qkv: 256x256
    (6223, 3072, 768, 2, 64),    # info-sharing fc1: 320x256
    (5838, 1152, 384, 0, 64),    # DA3-Small C2 qkv
    (1297, 1536, 384, 2, 64),    # DA3-Small C1 fc1
    (2074, 3072, 1024, 0, 64),   # MapAnything C3 encoder qkv
    (1400, 4608, 1536, 0, 128),  # reference-dims MapAnything qkv (128-column groups)
    (100, 256, 1024, 1, 64),     # would split K: runs unsplit (a row's statistics need all of K); ragged rows
    (333, 640, 192, 0, 64),      # 128-row tiles, ragged rows, three partials a row
    (64, 64, 64, 0, 64),         # one tile, one k-tile, one partial
]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("M,N,K,act,group", LN_CONSUMER_CASES)
def test_gemm_folded_layernorm_matches_torch(ctx, dtype, M, N, K, act, group):
    """act(LN(x) W^T + b) from the un-normalised rows, their statistics (ln_stats kernel) and the
    folded weights, rows with a non-zero mean so that the mean term matters: (1) the epilogue
    algebra against fp64 on the same rounded operands; (2) the whole fold against torch's
    LayerNorm and linear in fp64 (bf16, f16: the rounding of x and of W * gamma)."""
    report("gemm_ln", dtype=dtype, M=M, N=N, K=K, act=act, group=group)
    code, tdt = _dt(dtype)
    g = torch.Generator().manual_seed(M + 5 * N + 11 * K)
    x = torch.randn(M, K, generator=g) + 0.7 * torch.randn(M, 1, generator=g)
    gamma = 1 + 0.2 * torch.randn(K, generator=g)
    beta = 0.1 * torch.randn(K, generator=g)
    Wl = torch.randn(N, K, generator=g) * 0.05
    bl = torch.randn(N, generator=g) * 0.1
    Wf = (Wl * gamma).to(tdt)           # folded, as stored
    c1 = Wf.double().sum(1).float()
    c2 = (bl.double() + Wl.double() @ beta.double()).float()
    ldw = (K + 63) // 64 * 64
    Wp = torch.zeros(N, ldw, dtype=tdt)
    Wp[:, :K] = Wf
    dx = x.cuda()
    stats = torch.empty(M, K // group, 2, device="cuda")
    copy = torch.empty(M, K, dtype=tdt, device="cuda") if dtype != "f32" else None
    dW, dc1, dc2 = Wp.cuda(), c1.cuda(), c2.cuda()
    out = torch.empty(M, N, device="cuda")
    torch.cuda.synchronize()
    ctx.kernel_ln_stats(dx.data_ptr(), M, K, group, stats.data_ptr(), code, copy.data_ptr() if copy is not None else 0)
    A = copy if copy is not None else dx
    ctx.kernel_gemm_ln(code, A.data_ptr(), M, K, dW.data_ptr(), N, ldw, dc2.data_ptr(), act, out.data_ptr(), True,
                       ln_in=stats.data_ptr(), c1=dc1.data_ptr(), eps=1e-6, group=group)
    ctx.synchronize()
    st = stats.cpu().double()
    ref_st = _group_sums(x, group)
    assert torch.allclose(st, ref_st, rtol=1e-5, atol=1e-3), (st - ref_st).abs().max()
    if copy is not None:
        assert torch.equal(copy.cpu(), x.to(tdt))
    # (1) same operands: rstd * (x~ Wf^T - mean c1) + c2, statistics of the fp32 rows
    mean = ref_st[:, :, 0].sum(1, keepdim=True) / K
    rstd = 1 / torch.sqrt(ref_st[:, :, 1].sum(1, keepdim=True) / K - mean * mean + 1e-6)
    xs = x.to(tdt).double()
    act_fn = {0: lambda t: t, 1: torch.relu, 2: torch.nn.functional.gelu}[act]
    ref = act_fn(rstd * (xs @ Wf.double().T - mean * c1.double()[None]) + c2.double())
    got = out.cpu().double()
    err = (got - ref).abs().max().item() / (ref.abs().max().item() + 1e-12)
    # (2) the fold against LayerNorm -> linear
    true = act_fn(torch.nn.functional.layer_norm(x.double(), (K,), gamma.double(), beta.double(), 1e-6)
                  @ Wl.double().T + bl.double())
    err2 = (got - true).abs().max().item() / (true.abs().max().item() + 1e-12)
    report("gemm_ln.err", same_operands=f"{err:.2e}", vs_layer_norm=f"{err2:.2e}")
    assert err < 2e-5, err
    assert err2 < _tol(dtype, 1e-5, 2e-2, 4e-3), err2


def test_gemm_split_k_repeat(ctx):
    """Split-K launches (fp32 partials in the context's workspace, summed in slice order by a
    reduce kernel): each call starts from an output full of NaN, and calls of other shapes in
    between reuse the same workspace; every call must write every output, bit for bit the first
    call's result."""
    outs = {}
    shapes = [(1297, 384, 1536, "f32"), (100, 256, 4096, "bf16"), (777, 64, 2048, "f32"), (1297, 384, 1536, "f32"),
              (300, 1001, 2048, "bf16"), (100, 256, 4096, "f16"), (100, 256, 4096, "bf16"), (300, 1001, 2048, "f16")]
    for M, N, K, dtype in shapes:
        code, tdt = _dt(dtype)
        g = torch.Generator().manual_seed(M + N + K)
        A = torch.randn(M, K, generator=g).to(tdt).cuda()
        ldw = (K + 63) // 64 * 64
        Wm = torch.zeros(N, ldw)
        Wm[:, :K] = torch.randn(N, K, generator=g) * 0.05
        dW = Wm.to(tdt).cuda()
        b = torch.randn(N, generator=g).cuda()
        out = torch.full((M, N), float("nan"), dtype=tdt, device="cuda")
        torch.cuda.synchronize()
        ctx.kernel_gemm(code, A.data_ptr(), M, K, dW.data_ptr(), N, ldw, b.data_ptr(), 1, out.data_ptr(), False)
        ctx.synchronize()
        got = out.cpu()
        report("gemm.splitk.repeat", M=M, N=N, K=K, dtype=dtype)
        assert torch.isfinite(got.float()).all()
        key = (M, N, K, dtype)
        if key in outs:
            assert torch.equal(outs[key], got)
        else:
            ref = torch.relu(A.cpu().double() @ dW.cpu().double()[:, :K].T + b.cpu().double())
            err = ((got.double() - ref).abs().max() / ref.abs().max()).item()
            assert err < (1e-5 if dtype == "f32" else 1e-2), err
            outs[key] = got


LN_PRODUCER_CASES = [
    # (M, N, K, group): proj / fc2 residual epilogues
    (6222, 1024, 1024, 64),   # MapAnything encoder proj: 256x128 tiles
    (6222, 1024, 4096, 64),   # encoder fc2
    (6223, 768, 768, 64),     # info proj: 192x128 tiles (32-column waves: sums meet in LDS)
    (6223, 768, 3072, 64),    # info fc2
    (5838, 384, 1536, 64),    # DA3-Small C2 fc2: 128x128 tiles
    (1297, 384, 1536, 64),    # DA3-Small C1 fc2: split-K, statistics from the reduce kernel
    (1297, 1536, 1536, 128),  # split-K, 128-column groups (16-lane sums in the reduce kernel)
    (1400, 1536, 1536, 128),  # reference-dims MapAnything proj (128-column groups)
    (6222, 4096, 1024, 128),  # 400 tiles of 256x256 (1.56 rounds), 32 groups a row
    (200, 128, 64, 64),       # one row tile, ragged
]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("M,N,K,group", LN_PRODUCER_CASES)
def test_gemm_residual_statistics(ctx, dtype, M, N, K, group):
    """out = res + gamma * (A W^T + b) in fp32, the (sum, sum of squares) of every output row per
    group of columns, and the output rows in the GEMM's dtype, bit for bit the stored rows rounded."""
    report("gemm_resln", dtype=dtype, M=M, N=N, K=K, group=group)
    code, tdt = _dt(dtype)
    g = torch.Generator().manual_seed(3 * M + N + 7 * K)
    A = torch.randn(M, K, generator=g).to(tdt)
    ldw = (K + 63) // 64 * 64
    Wm = torch.zeros(N, ldw)
    Wm[:, :K] = torch.randn(N, K, generator=g) * 0.05
    Wm = Wm.to(tdt)
    bias = torch.randn(N, generator=g)
    gam = torch.rand(N, generator=g) + 0.5
    res = torch.randn(M, N, generator=g)
    dA, dW, db, dg, dr = A.cuda(), Wm.cuda(), bias.cuda(), gam.cuda(), res.cuda()
    out = torch.empty(M, N, device="cuda")
    stats = torch.full((M, N // group, 2), float("nan"), device="cuda")
    copy = torch.empty(M, N, dtype=tdt, device="cuda")
    torch.cuda.synchronize()
    ctx.kernel_gemm_ln(code, dA.data_ptr(), M, K, dW.data_ptr(), N, ldw, db.data_ptr(), 0, out.data_ptr(), True,
                       gamma=dg.data_ptr(), res=dr.data_ptr(), ln_out=stats.data_ptr(), copy=copy.data_ptr(),
                       group=group)
    ctx.synchronize()
    ref = res.double() + gam.double() * (A.double() @ Wm[:, :K].double().T + bias.double())
    got = out.cpu()
    err = (got.double() - ref).abs().max().item() / (ref.abs().max().item() + 1e-12)
    st = stats.cpu().double()
    ref_st = _group_sums(got, group)  # the statistics are of the stored fp32 outputs
    scale = _group_sums(got.abs(), group)
    st_err = ((st - ref_st).abs() / (scale + 1e-6)).max().item()
    report("gemm_resln.err", out=f"{err:.2e}", stats=f"{st_err:.2e}")
    assert err < (1e-5 if dtype == "f32" else 2e-5), err
    assert st_err < 1e-5, st_err
    assert torch.equal(copy.cpu(), got.to(tdt))


@pytest.mark.parametrize("dtype", DTYPES)
def test_gemm_operand_beyond_2gib(ctx, dtype):
    """An A operand of 2 GiB or more leaves the 32-bit buffer offsets of the MFMA path: the GEMM
    runs on the register-staged kernel (gemm.hip gemm_kernel, 64-bit addresses). Rows sampled
    at the start, across the 2 GiB boundary and at the ragged end against fp64."""
    code, tdt = _dt(dtype)
    es = 4 if dtype == "f32" else 2
    K, N = 1024, 96
    M = (1 << 31) // (K * es) + 37
    report("gemm.2gib", dtype=dtype, M=M, N=N, K=K, A_bytes=M * K * es)
    g = torch.Generator(device="cuda").manual_seed(7)
    A = torch.randn(M, K, device="cuda", dtype=tdt, generator=g)
    Wm = torch.zeros(N, K, dtype=tdt)
    Wm[:, :] = (torch.randn(N, K, generator=torch.Generator().manual_seed(8)) * 0.05).to(tdt)
    b = torch.randn(N, generator=torch.Generator().manual_seed(9))
    dW, db = Wm.cuda(), b.cuda()
    out = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    ctx.kernel_gemm(code, A.data_ptr(), M, K, dW.data_ptr(), N, K, db.data_ptr(), 1, out.data_ptr(), True)
    ctx.synchronize()
    # contiguous row ranges copied to the host (torch's gather kernel is not used on a tensor
    # this large: its index arithmetic faults past 2 GiB)
    half = (1 << 31) // (K * es)
    err = 0.0
    for r0, r1 in ((0, 64), (half - 64, half + 64), (M - 64, M)):
        ref = torch.relu(A[r0:r1].cpu().double() @ Wm.double().T + b.double())
        got = out[r0:r1].cpu().double()
        err = max(err, ((got - ref).abs().max() / ref.abs().max()).item())
    report("gemm.2gib.err", err=f"{err:.2e}")
    assert err < 1e-5, err
    del A, out
    torch.cuda.empty_cache()


def test_conv_input_beyond_2gib(ctx):
    """A bf16 convolution whose input map is 2 GiB (2 views of 512 x 512 x 2048) runs on the
    register-staged kernel; output pixels at the corners, edges and the map's far end against
    fp64 sums over their 3 x 3 neighbourhoods (zero padding)."""
    code, tdt = _dt("bf16")
    V, H, W, Cin, Cout = 2, 512, 512, 2048, 48
    report("conv2d.2gib", V=V, H=H, W=W, Cin=Cin, Cout=Cout, in_bytes=V * H * W * Cin * 2)
    g = torch.Generator(device="cuda").manual_seed(11)
    x = torch.randn(V, H, W, Cin, device="cuda", dtype=tdt, generator=g)
    K = 9 * Cin
    w = (torch.randn(Cout, 3, 3, Cin, generator=torch.Generator().manual_seed(12)) * 0.02).to(tdt)
    b = torch.randn(Cout, generator=torch.Generator().manual_seed(13))
    dw, db = w.reshape(Cout, K).contiguous().cuda(), b.cuda()
    out = torch.full((V, H, W, Cout), float("nan"), dtype=tdt, device="cuda")
    torch.cuda.synchronize()
    ctx.kernel_conv2d(code, x.data_ptr(), V, H, W, Cin, dw.data_ptr(), Cout, K, 3, 1, db.data_ptr(), 0, 0, 0,
                      out.data_ptr())
    ctx.synchronize()
    pix = [(0, 0, 0), (0, 0, W - 1), (0, H - 1, 7), (0, 255, 300), (1, 0, 0), (1, 311, 0), (1, 200, 511),
           (1, H - 1, W - 1), (1, H - 2, W - 3)]
    wd = w.double()
    err = 0.0
    for v, y, xx in pix:
        acc = b.double().clone()
        for ky in range(3):
            for kx in range(3):
                iy, ix = y + ky - 1, xx + kx - 1
                if 0 <= iy < H and 0 <= ix < W:
                    acc += wd[:, ky, kx, :] @ x[v, iy, ix].cpu().double()
        got = out[v, y, xx].cpu().double()
        err = max(err, ((got - acc).abs() / (acc.abs() + 0.05 * acc.abs().max())).max().item())
    report("conv2d.2gib.err", err=f"{err:.2e}")
    assert err < 1e-2, err
    del x, out
    torch.cuda.empty_cache()
