"""BASELINE config 4 at its real size: the FP8 e4m3fn W8A8 linears of one decoder layer on
8 x 1024 packed prefill tokens (M = 8192), FP8Linear (kernels/fp8_linear.py:66-126) against
the oracle on the same quantised operands.

Shapes (K -> N): QKV 1536 -> 2048 (with the q|k|v bias), O 1536 -> 1536, gate/up
1536 -> 17920, down 8960 -> 1536; x ~ N(0, 1) fp16, W ~ N(0, 0.02) fp16 (config 4).  At
M = 8192 every config-4 shape runs a persistent grid of 256-row big tiles (gate/up: 32 x 70
tiles of 256 x 256 on 256 workgroups, 9 rounds; O and down 256 tiles of 256 x 192, one
per CU); the 256 x 128 pipeline takes the down shape at M = 4096 (big tiles would fill half
the grid) and a ragged M (a partial tile in the last round); K < 512 takes the
one-tile-per-workgroup kernel.  ``omni_fp8_gemm_plan`` names the kernel and grid each case
runs, so the test states which path it covered.

The oracle's product is computed for 8 rows of every 256-row block (one row in each of
the four 64-row wave bands, several 16-row sub-tiles and lane positions) and every column:
every output tile of every round is compared.  All M rows are checked against a
size-independent property: sum_n y[m, n] equals sa[m] * (xq[m] . (Wq^T sw)) up to the
roundings of each term."""

import pytest
import torch

from oracle import qwen2_ref as ref

pytestmark = pytest.mark.gpu

KIND = {0: "one tile per workgroup", 1: "pipelined 256x128 persistent",
        2: "persistent 256x256 tiles", 3: "persistent 256x192 tiles"}
COLS = {0: 128, 1: 128, 2: 256, 3: 192}
BLOCK_ROWS = (0, 17, 63, 98, 133, 228, 239, 255)    # within each 256-row block


def say(msg):
    print(f"[gpu-test] {msg}", flush=True)


def f16(shape, seed, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).to(torch.float16)


def sample_rows(M):
    rows = sorted({b + r for b in range(0, M, 256) for r in BLOCK_ROWS if b + r < M} | {M - 1})
    return torch.tensor(rows, dtype=torch.long)


def plan(M, N, K):
    from omniserver_amd._lib import lib
    import ctypes
    g = ctypes.c_int(0)
    kind = lib().omni_fp8_gemm_plan(M, N, K, ctypes.byref(g))
    return kind, g.value


def abs_product(xq, sa, wq, sw):
    return (xq.float().abs() @ wq.float().abs().t()) * sa.view(-1, 1) * sw.view(1, -1)


CASES = [
    # name, M, K, N, bias
    ("qkv", 8192, 1536, 2048, True),
    ("o", 8192, 1536, 1536, False),
    ("gate_up", 8192, 1536, 17920, False),
    ("gate_up biased", 8192, 1536, 17920, True),   # 192-column tail tiles with biases
    ("down", 8192, 8960, 1536, False),
    ("256-wide", 8192, 4096, 2048, True),
    ("down half grid", 4096, 8960, 1536, False),
    ("gate_up ragged", 8192 + 100, 1536, 17920, False),
    ("down ragged", 2000, 8960, 1536, True),
    ("short K", 1000, 384, 2048, True),
]


@pytest.mark.parametrize("name,M,K,N,bias", CASES, ids=[c[0] for c in CASES])
def test_fp8_config4_linear(gpu, name, M, K, N, bias):
    from omniserver_amd.linear import FP8Linear
    kind, grid = plan(M, N, K)
    tiles = -(-M // (256 if kind else 128)) * (N // COLS[kind])
    say(f"fp8 {name}: M={M} K={K} N={N} bias={bias} -> {KIND[kind]}, grid {grid}, "
        f"{tiles} tiles ({-(-tiles // grid)} rounds)")
    W = f16((N, K), 400 + N % 97, 0.02)
    b = f16((N,), 401, 0.02) if bias else None
    x = f16((M, K), 402 + K % 89)
    lin = FP8Linear(W.to(gpu), None if b is None else b.to(gpu), rowwise=True)
    y = lin(x.to(gpu)).cpu()
    torch.cuda.synchronize()
    wq, sw = ref.fp8_weight_rowwise(W.float())
    assert torch.equal(lin.weight_fp8.cpu(), wq.view(torch.uint8))
    xq, sa = ref.quant_fp8(x.float())

    # every tile: sampled rows, all columns, against the oracle
    rows = sample_rows(M)
    e = ref.fp8_linear_rowwise(xq[rows], sa[rows], wq, sw, None if b is None else b.float())
    e0 = ref.fp8_linear_rowwise(xq[rows], sa[rows], wq, sw, None)
    yc = y[rows].float()
    d = (yc - e).abs()
    tol = (e0.abs() * 2.0 ** -7 + e.abs() * 2.0 ** -10
           + abs_product(xq[rows], sa[rows], wq, sw) * 2.0 ** -14)
    assert (d <= tol + 1e-6).all(), (d - tol).max().item()
    same = (d == 0).float().mean().item()
    assert same > 0.95, same

    # every row: the row sum against the closed form (each output within one bf16 step,
    # one fp16 step and the bias rounding of its exact value)
    exact_sum = sa.view(-1) * (xq.float() @ (wq.float().t() @ sw))
    if b is not None:
        exact_sum = exact_sum + b.float().sum()
    ysum = y.float().sum(1)
    ymag = y.float().abs().sum(1)
    bound = (ymag * (2.0 ** -8 + 2.0 ** -10) + 1e-3
             + (xq.float().abs() @ (wq.float().abs().t() @ sw)) * sa.view(-1) * 2.0 ** -14)
    assert ((ysum - exact_sum).abs() <= bound).all(), ((ysum - exact_sum).abs() - bound).max()
    say(f"fp8 {name}: {len(rows)} sampled rows x {N} columns, {100 * same:.2f}% bit-equal; "
        f"{M} row sums within bounds")


def test_fp8_prequant_bias_bf16(gpu):
    """forward_prequant with a bias (fp8_linear.py:99-108): bf16 product + bias.to(bf16) as
    a bf16 add, at a size that runs the persistent pipelined kernel."""
    from omniserver_amd import fused_ops as F
    from omniserver_amd.linear import FP8Linear
    M, H, N = 1024, 1536, 4096
    say(f"fp8 prequant + bias M={M} N={N}")
    x, r = f16((M, H), 410), f16((M, H), 411)
    w = torch.ones(H, dtype=torch.float16)
    W = f16((N, H), 412, 0.02)
    b = f16((N,), 413, 0.05)
    lin = FP8Linear(W.to(gpu), b.to(gpu), rowwise=True)
    q, s, _ = F.add_rms_norm_fp8(x.to(gpu), r.to(gpu), w.to(gpu), 1e-6)
    y = lin.forward_prequant(q, s)
    torch.cuda.synchronize()
    assert y.dtype == torch.bfloat16
    wq, sw = ref.fp8_weight_rowwise(W.float())
    qc = q.cpu().view(torch.float8_e4m3fn)
    e = ref.fp8_linear_prequant(qc, s.cpu(), wq, sw, b.float())
    e0 = ref.fp8_linear_prequant(qc, s.cpu(), wq, sw, None)
    d = (y.cpu().float() - e).abs()
    tol = (e0.abs() + e.abs()) * 2.0 ** -7 + abs_product(qc, s.cpu(), wq, sw) * 2.0 ** -14
    assert (d <= tol + 1e-6).all(), (d - tol).max().item()
    assert (d == 0).float().mean().item() > 0.95


def test_bf16_rounding_exhaustive(gpu):
    """The FP8 epilogues round to bf16 with the device's packed conversion: on every one of
    the 2^32 float bit patterns it equals the integer round-to-nearest-even with quieted NaNs
    (the rounding of the reference's bf16 outputs), NaN inputs included."""
    from omniserver_amd._lib import call, ptr, stream
    say("bf16 rounding: all 2^32 float inputs")
    mism = torch.zeros(2, device=gpu, dtype=torch.int64)
    call("omni_bf16_rne_check", ptr(mism), stream())
    torch.cuda.synchronize()
    assert mism.tolist() == [0, 0]
