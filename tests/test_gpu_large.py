"""Tensors past 2^31 elements: one launch per family on the benchmarked hw
variant and tiles, with inputs drawn on the GPU, checked against the oracle
on sampled rows on both sides of element 2^31 (where a 32-bit index would
wrap) and at the ends. Each case allocates 9-18 GB of HBM and frees it
before the next."""

import math

import pytest
import torch

import oracle
from enzyme_amd import hip

pytestmark = pytest.mark.gpu

TWO31 = 1 << 31


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"


@pytest.fixture(autouse=True)
def _free():
    yield
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def _gen(seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return g


def _launch(name, variant, tiles, dims, inputs):
    print(f"large {name} v{variant} {tuple(tiles)} dims {dims}", flush=True)
    ln = hip.Launcher(name, variant, tiles, dims, inputs)
    ln.launch()
    torch.cuda.synchronize()
    return ln.outputs


def test_rmsnorm_rows_past_2_31_elements():
    m, n = TWO31 // 4096 + 3, 4096
    assert m * n > TWO31
    g = _gen(1)
    x = torch.randn((m, n), generator=g, device="cuda").to(torch.bfloat16)
    w = (1.0 + 0.1 * torch.randn((n,), generator=g, device="cuda")).to(torch.bfloat16)
    (y,) = _launch("rmsnorm_weighted", 0, (1, 8), [m, n], [x, w])
    rows = torch.tensor([0, 1, m // 2, TWO31 // n - 1, TWO31 // n, TWO31 // n + 1, m - 1])
    want = oracle.ORACLE["rmsnorm_weighted"](x[rows.cuda()].cpu(), w.cpu())
    torch.testing.assert_close(y[rows.cuda()].float().cpu(), want, rtol=1e-2, atol=1e-2)


def test_cumsum_rows_past_2_31_elements():
    m, n = TWO31 // 131072 + 1, 131072
    assert m * n > TWO31
    g = _gen(2)
    p = torch.rand((m, n), generator=g, device="cuda")
    p /= p.sum(dim=1, keepdim=True)
    rows = torch.tensor([0, m // 2, TWO31 // n - 1, TWO31 // n, m - 1])
    want = oracle.ORACLE["cumsum_probs"](p[rows.cuda()].cpu())
    for variant, tiles in ((2, (4, 8)), (0, (16, 4))):
        (y,) = _launch("cumsum_probs", variant, tiles, [m, n], [p])
        torch.testing.assert_close(y[rows.cuda()].cpu(), want, rtol=1e-5, atol=1e-9)
        del y


def test_rope_tokens_past_2_31_elements():
    b, s, hq, hkv, d = 1, TWO31 // (32 * 128) + 1, 32, 8, 128
    assert b * s * hq * d > TWO31
    g = _gen(3)
    q = torch.randn((b, s, hq, d), generator=g, device="cuda").to(torch.bfloat16)
    k = torch.randn((b, s, hkv, d), generator=g, device="cuda").to(torch.bfloat16)
    cos = torch.rand((s, d), generator=g, device="cuda") * 2 - 1
    sin = torch.rand((s, d), generator=g, device="cuda") * 2 - 1
    qo, ko = _launch("rope_llama3", 1, (16, 8), [b, s, hq, hkv, d], [q, k, cos, sin])
    toks = torch.tensor([0, 1, s // 2, TWO31 // (hq * d) - 1, s - 1]).cuda()
    wq, wk = oracle.ORACLE["rope_llama3"](q[:, toks].cpu(), k[:, toks].cpu(), cos[toks].cpu(), sin[toks].cpu())
    torch.testing.assert_close(qo[:, toks].float().cpu(), wq, rtol=1e-2, atol=1e-2)
    torch.testing.assert_close(ko[:, toks].float().cpu(), wk, rtol=1e-2, atol=1e-2)


def test_matmul_a_past_2_31_elements():
    m, n, k = 131072, 64, 16392
    assert m * k > TWO31
    g = _gen(4)
    a = (torch.randn((m, k), generator=g, device="cuda") / math.sqrt(k)).to(torch.bfloat16)
    w = torch.randn((k, n), generator=g, device="cuda").to(torch.bfloat16)
    tiles = next(t for t in ((2, 1, 8), (2, 1, 4), (1, 1, 4), (1, 1, 1))
                 if hip.check("matmul", 1, t, [m, n, k], [hip.AXON_BF16] * 2)[0] == hip.AXON_OK)
    (c,) = _launch("matmul", 1, tiles, [m, n, k], [a, w])
    rows = torch.tensor([0, m // 2, TWO31 // k, m - 1]).cuda()
    want = oracle.ORACLE["matmul"](a[rows].cpu(), w.cpu())
    torch.testing.assert_close(c[rows].float().cpu(), want, rtol=1e-2, atol=1e-2)


def test_attention_heads_past_2_31_elements():
    b, h, s, d = 1, 128, 131080, 128
    assert b * h * s * d > TWO31
    g = _gen(5)
    q, k, v = (torch.randn((b, h, s, d), generator=g, device="cuda").to(torch.bfloat16) for _ in range(3))
    (o,) = _launch("attention_causal", 2, (2, 2, 1, 1), [b, h, s, d], [q, k, v])
    # Query rows of the last head whose elements lie past 2^31, and the
    # first rows of head 0.
    first_past = TWO31 // d - (h - 1) * s
    for head, rows in ((0, [0, 1, 777]), (h - 1, [first_past - 1, first_past, s - 1])):
        for r in rows:
            qr = q[0, head, r:r + 1].float().cpu()
            kr, vr = k[0, head, :r + 1].float().cpu(), v[0, head, :r + 1].float().cpu()
            want = torch.softmax(qr @ kr.T / math.sqrt(d), dim=-1) @ vr
            torch.testing.assert_close(o[0, head, r:r + 1].float().cpu(), want, rtol=1e-2, atol=1e-2,
                                       msg=lambda m_, hh=head, rr=r: f"head {hh} row {rr}: {m_}")
