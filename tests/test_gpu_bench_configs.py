"""GPU parity of exactly what bench.py times: for every workload row of
bench.CONFIGS, the same spec, sizes, hw variant and tile tuple, at full size,
against the oracle at the row's own tolerance (rtol = atol = 1e-2 for bf16
outputs, rtol 1e-5 / atol 0 for the fp32 scan of probabilities, 2e-2 for
qkv_cte). The test ids name the tuple, e.g. `rope_llama3-v0-4x1`."""

import pytest
import torch

import bench
from tests._gpu import check_parity

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"


def _id(cfg):
    return f"{cfg['spec']}-v{cfg['variant']}-{'x'.join(map(str, cfg['tiles']))}"


@pytest.mark.parametrize("cfg", bench.CONFIGS, ids=[_id(c) for c in bench.CONFIGS])
def test_benchmarked_instantiation(cfg):
    print(f"bench row {_id(cfg)} sizes {cfg['sizes']}", flush=True)
    assert check_parity(cfg["spec"], cfg["sizes"], rtol=cfg["rtol"], atol=cfg["atol"],
                        variants=[cfg["variant"]], tiles=cfg["tiles"]) == 1
