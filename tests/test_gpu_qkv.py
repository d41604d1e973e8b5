"""GPU parity for qkv_cte (residual add -> RMSNorm with eps -> projection)
through the C ABI, against the fp32 oracle on the spec's own seeded inputs.

Tolerances: bf16 cases are held to rtol = atol = 2e-2, tighter than the
reference's bf16 case tolerance (rtol 5e-2, atol 1.5e-1, eval/sizes.json);
fp32 cases to the reference's rtol = atol = 1e-3 (the split-precision GEMM
keeps about 1e-5). Shapes: the reference's vision_l4 (ragged m = 578,
n = 264) and llama405b_1k cases in both dtypes, over a diverse selection of
legal tile tuples in every hw variant (split-K and single-pass schedules;
hw variants 2 and 3, the fused residual sum, take bf16 only; hw variant 3
counts TILES_IN_BLOCK_N in units of 256 columns),
plus small edge shapes (one row, k = 8, m = 0). The llama70b case
(16384 x 512 x 8192) is checked against torch's fp32 product on the GPU."""

import numpy as np
import pytest
import torch

import oracle
from enzyme_amd import hip
from tests._gpu import check_parity
from tests._specs import spec_inputs, to_device

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"


@pytest.mark.parametrize("sizes", [(578, 264, 1408), (1024, 512, 16384)], ids=["vision_l4", "llama405b_1k"])
def test_qkv_bf16_reference_cases(sizes):
    assert check_parity("qkv_cte", sizes, rtol=2e-2, atol=2e-2, budget=6)


@pytest.mark.parametrize("sizes", [(578, 264, 1408), (1024, 512, 16384)], ids=["vision_l4", "llama405b_1k"])
def test_qkv_fp32_reference_cases(sizes):
    assert check_parity("qkv_cte", sizes, rtol=1e-3, atol=1e-3, budget=6, dtype="float32", variants=(0, 1))


@pytest.mark.parametrize("dtype", [None, "float32"], ids=["bf16", "fp32"])
@pytest.mark.parametrize("sizes", [(1, 8, 8), (77, 136, 520), (130, 72, 64)])
def test_qkv_edge_shapes(sizes, dtype):
    tol = 1e-3 if dtype == "float32" else 2e-2
    variants = (0, 1) if dtype == "float32" else None
    assert check_parity("qkv_cte", sizes, rtol=tol, atol=tol, dtype=dtype, budget=4, variants=variants)


@pytest.mark.parametrize("variant", [2, 3])
def test_qkv_fused_variant_refuses_fp32(variant):
    st, why = hip.check("qkv_cte", variant, (2, 2, 4), [256, 128, 4096], [hip.AXON_F32] * 4)
    assert st == hip.AXON_EDTYPE and "bf16" in why


def test_qkv_zero_rows_is_a_no_op():
    """m = 0 launches nothing and writes nothing. The C ABI refuses null
    pointers, so the empty operands are zero-row views of live buffers."""
    spec, dims, host = spec_inputs("qkv_cte", (2, 64, 64))
    x, mp, ap, w = to_device(host)
    out = torch.full((2, 64), 7.0, device="cuda", dtype=torch.bfloat16)
    ln = hip.Launcher("qkv_cte", 0, (1, 1, 1), [0, 64, 64], [x[:0], mp[:0], ap[:0], w], outputs_=[out[:0]])
    ln.launch()
    torch.cuda.synchronize()
    assert torch.all(out == 7.0)


@pytest.mark.parametrize("variant", [0, 1, 2, 3])
def test_qkv_llama70b_against_torch_fp32(variant):
    """Full llama70b shape (16384 x 512 x 8192, bf16 inputs), split-K tiles:
    compared with torch's fp32 restatement of the reference formula on the
    GPU (h summed in fp32, mean form with eps, fp32 product)."""
    m, n, k = 16384, 512, 8192
    g = torch.Generator(device="cuda").manual_seed(3)
    x, mp, ap = (torch.randn(m, k, device="cuda", generator=g).to(torch.bfloat16) for _ in range(3))
    w = (torch.randn(k, n, device="cuda", generator=g) / np.sqrt(k)).to(torch.bfloat16)
    ln = hip.Launcher("qkv_cte", variant, (2, 2, 8), [m, n, k], [x, mp, ap, w])
    ln.launch()
    torch.cuda.synchronize()
    h = (x.float() + mp.float()) + ap.float()
    ref = (h * torch.rsqrt((h * h).mean(dim=-1, keepdim=True) + 1e-6)) @ w.float()
    torch.testing.assert_close(ln.outputs[0].float(), ref, rtol=2e-2, atol=2e-2)


@pytest.mark.parametrize(("dtype", "variant"), [(None, 1), (None, 2), (None, 3), ("float32", 1)],
                         ids=["bf16-v1", "bf16-v2", "bf16-v3", "fp32-v1"])
def test_qkv_repeated_launches_bit_identical(dtype, variant):
    """Split-K sums its partials in a fixed order and the prep pass is
    elementwise, so relaunching over the same workspace reproduces the
    output bit for bit."""
    spec, dims, host = spec_inputs("qkv_cte", (256, 128, 4096), dtype=dtype)
    dev = to_device(host)
    ln = hip.Launcher("qkv_cte", variant, (2, 2, 4), [256, 128, 4096], dev)
    ln.launch()
    torch.cuda.synchronize()
    first = ln.outputs[0].clone()
    for _ in range(5):
        ln.launch()
    torch.cuda.synchronize()
    assert torch.equal(first, ln.outputs[0])
    ref = oracle.qkv_cte(*[t.cpu() for t in dev])
    torch.testing.assert_close(first.float().cpu(), ref, rtol=2e-2, atol=2e-2)


@pytest.mark.parametrize(("sizes", "dtype", "variant"),
                         [((16384, 640, 12288), torch.bfloat16, 2), ((16384, 640, 12288), torch.bfloat16, 1),
                          ((16384, 640, 12288), torch.bfloat16, 3),
                          ((8192, 512, 16384), torch.bfloat16, 2), ((8192, 512, 16384), torch.bfloat16, 3),
                          ((8192, 512, 16384), torch.float32, 1),
                          ((16384, 512, 8192), torch.float32, 0), ((16384, 640, 12288), torch.float32, 1)],
                         ids=["mistral123b-v2", "mistral123b-v1", "mistral123b-v3", "llama405b_8k-v2",
                              "llama405b_8k-v3", "llama405b_8k_fp32-v1", "llama70b_fp32-v0", "mistral123b_fp32-v1"])
def test_qkv_large_reference_cases(sizes, dtype, variant):
    """The reference's large cases (mistral123b, n = 640: a ragged last N tile
    at 128 or 256 columns; llama405b_8k; the fp32 llama70b / mistral123b /
    llama405b_8k) at full size, inputs drawn on the GPU, against torch's fp32
    restatement of the reference formula, at the reference's tolerances
    (bf16: rtol 5e-2, atol 1.5e-1; fp32: 1e-3). hw variant 3's (2, 2, 8) is a
    128 x 512 tile: at n = 640 its second N tile holds 128 live columns."""
    m, n, k = sizes
    g = torch.Generator(device="cuda").manual_seed(5)
    x, mp, ap = (torch.randn(m, k, device="cuda", generator=g).to(dtype) for _ in range(3))
    w = (torch.randn(k, n, device="cuda", generator=g) / np.sqrt(k)).to(dtype)
    codes = [hip.dtype_code(x)] * 4
    tiles = (2, 2, 8)
    assert hip.check("qkv_cte", variant, tiles, [m, n, k], codes)[0] == hip.AXON_OK
    ln = hip.Launcher("qkv_cte", variant, tiles, [m, n, k], [x, mp, ap, w])
    ln.launch()
    torch.cuda.synchronize()
    h = (x.float() + mp.float()) + ap.float()
    ref = (h * torch.rsqrt((h * h).mean(dim=-1, keepdim=True) + 1e-6)) @ w.float()
    tol = (1e-3, 1e-3) if dtype == torch.float32 else (5e-2, 1.5e-1)
    torch.testing.assert_close(ln.outputs[0].float(), ref, rtol=tol[0], atol=tol[1])
