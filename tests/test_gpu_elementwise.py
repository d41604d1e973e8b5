"""GPU parity for RoPE (split layout and token-major) and fused Adam.

Tolerances: rope at the reference's case tolerance rtol 7.8125e-3 /
atol 2e-2 (eval/sizes.json); rope_llama3 and bf16 Adam rtol = atol = 1e-2;
fp32 Adam rtol 1e-5 (its operations round in the reference's order, so the
result is expected to match bit for bit; the bar stays the stated 1e-5)."""

import pytest
import torch

from tests._gpu import check_parity

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"


@pytest.mark.parametrize("sizes", [(128, 4096), (128, 32768), (7, 33)])
def test_rope_split(sizes):
    assert check_parity("rope", sizes, rtol=7.8125e-3, atol=2e-2, budget=12 if sizes[1] > 10000 else 0)


@pytest.mark.parametrize("sizes", [(1, 4096, 32, 8, 128), (2, 17, 4, 2, 64), (1, 5, 3, 1, 6), (3, 5, 4, 2, 128)])
def test_rope_llama3(sizes):
    assert check_parity("rope_llama3", sizes, rtol=1e-2, atol=1e-2, budget=10)


@pytest.mark.parametrize("sizes", [(1, 4096, 32, 8, 128), (3, 5, 4, 2, 128), (2, 17, 4, 2, 64)])
def test_rope_llama3_token_groups(sizes):
    """hw variant 1 (token-aligned workgroups, cos/sin rows in LDS) at every
    tokens-per-workgroup count: ragged last workgroups, and positions that
    wrap inside one workgroup (b > 1 with s < 16)."""
    for tpb in (1, 2, 4, 8, 16):
        for w in (1, 4):
            assert check_parity("rope_llama3", sizes, rtol=1e-2, atol=1e-2, variants=[1], tiles=(w, tpb)) == 1


@pytest.mark.parametrize("sizes", [(128, 8192), (5, 37)])
def test_fused_adam_bf16(sizes):
    assert check_parity("fused_adam", sizes, rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("sizes", [(128, 8192), (5, 37)])
def test_fused_adam_fp32(sizes):
    assert check_parity("fused_adam", sizes, rtol=1e-5, atol=1e-7, dtype="float32")
