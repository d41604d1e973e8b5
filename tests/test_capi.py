"""The C ABI of libaxon_hip.so on the host: the library loads without a
GPU, exports every symbol include/axon_hip.h declares, its registry covers
every spec package, and the host-only entry points (describe, manifest,
outputs, check, workspace) answer without touching the HIP runtime."""

import re
from itertools import product

import pytest

from enzyme_amd import hip
from enzyme_amd.bench_runner import _compile_one_variant
from enzyme_amd.emit import variant_module_text
from tests._specs import KERNELS, REPO, load_spec

HEADER = REPO / "include" / "axon_hip.h"
SPECS = sorted(p.name for p in KERNELS.iterdir() if (p / "__init__.py").is_file())


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(axon_[a-z_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    names = declared_symbols()
    assert names and set(names) == set(hip.EXPORTED_SYMBOLS)
    lib = hip.lib()
    for n in names:
        assert hasattr(lib, n), n


def test_registry_covers_every_spec_package():
    assert sorted(hip.kernel_names()) == SPECS
    for name in SPECS:
        spec = load_spec(name)
        n = hip.variant_count(name)
        assert n >= 1
        for v in range(n):
            d = hip.describe(name, v)
            assert d["tile_args"] == list(spec.tile_args)
            assert d["n_inputs"] == len(spec.input_specs)
            assert d["summary"]


def test_unknown_kernel_and_variant():
    assert hip.variant_count("no_such_kernel") == 0
    st, why = hip.check("no_such_kernel", 0, [1, 1], [1, 1], [0])
    assert st == hip.AXON_ENOKERNEL and "no_such_kernel" in why
    st, why = hip.check("rmsnorm", 7, [1, 1], [1, 1], [0])
    assert st == hip.AXON_ENOKERNEL
    st, _ = hip.check("rmsnorm", 0, [1, 1, 1], [1, 1], [0])
    assert st == hip.AXON_EARG
    st, _ = hip.check("rmsnorm", 0, [1, 1], [4, 64], [hip.AXON_F16])
    assert st == hip.AXON_EDTYPE


@pytest.mark.parametrize("name", SPECS)
def test_outputs_match_baseline_shapes(name):
    """Output descriptors agree with the spec's own baseline_op on small inputs."""
    import numpy as np

    from enzyme_amd.dtypes import to_f32_numpy
    from tests._specs import spec_inputs

    small = {"rope_llama3": (1, 8, 2, 1, 128), "attention_causal": (1, 2, 16, 128),
             "attention_nkilib": (16, 128), "silu_mlp": (16, 16, 16, 8), "fused_adam": (4, 16),
             "rope": (4, 16), "matmul": (8, 16, 16), "matmul_std002": (8, 16, 16),
             "rmsnorm_matmul": (8, 16, 16), "rmsnorm_matmul_eps": (8, 16, 16), "qkv_cte": (8, 16, 16),
             "softmax_mm": (8, 16, 16), "linear_attention": (8, 16, 16, 16), "attention": (16, 16, 16)}
    spec, dims, host = spec_inputs(name, small.get(name, (4, 64)))
    codes = [hip.AXON_BF16 if str(getattr(a, "dtype", "")).endswith("bfloat16") else hip.AXON_F32
             for a in host]
    outs = hip.outputs(name, [dims[d] for d in spec.dim_vars], codes)
    ref = spec.baseline_op(*[to_f32_numpy(a) for a in host])
    ref = ref if isinstance(ref, tuple) else (ref,)
    assert [o.shape for o in outs] == [tuple(np.shape(r)) for r in ref]


def test_manifest_literal_reads_back(tmp_path):
    from axon.candidate_filter import read_manifest

    spec = load_spec("matmul_std002")
    text = variant_module_text(spec, {"m": 1024, "n": 512, "k": 16384}, 0, 0, hip.AXON_BF16)
    p = tmp_path / "m.py"
    p.write_text(text)
    cons = read_manifest(p)
    assert cons == tuple(sorted(hip.manifest("matmul_std002", 0, [1024, 512, 16384], hip.AXON_BF16),
                                key=lambda c: c.tile_arg))
    k = {c.tile_arg: c for c in cons}["TILES_IN_BLOCK_K"]
    # The last K range may be ragged, so the K range need not divide k. The
    # occupancy box caps it at 2048: 128 x 128 tiles give 32 output tiles,
    # and 8 ranges of 2048 give them 256 workgroups.
    assert not k.require_divisible and k.tile_size == 256 and k.extent == 2048


# Families whose manifest admits the legal tuples inside an occupancy box
# (output tile and K range capped where the workgroup grid stops filling the
# chip); every other family's manifest admits exactly the legal tuples.
SPLITK_BOX = {"matmul", "matmul_std002", "rmsnorm_matmul", "rmsnorm_matmul_eps", "qkv_cte"}


def test_legal_tiles_are_a_subset_of_the_manifest():
    """Every tile tuple the library accepts passes the manifest the emitter
    writes (the filter never hides a legal instantiation), except, for the
    split-K GEMMs, tuples beyond the occupancy box: those fail only an extent
    cap, never divisibility, and the box keeps its (1, 1, 1) corner."""
    from axon.candidate_filter import rejection_reason

    cases = {"rmsnorm": [2048, 4096], "cumsum_probs": [64, 128256], "rope_llama3": [1, 4096, 32, 8, 128],
             "matmul": [1024, 512, 16384], "attention_causal": [1, 32, 4096, 128],
             "qkv_cte": [578, 264, 1408]}
    for name, dims in cases.items():
        spec = load_spec(name)
        dt = [hip.AXON_F32] if name == "cumsum_probs" else (
            [0, 0, 2, 2] if name == "rope_llama3" else [0] * len(spec.input_specs))
        for v in range(hip.variant_count(name)):
            cons = hip.manifest(name, v, dims, dt[0])
            legal = [t for t in product(spec.tile_options, repeat=len(spec.tile_args))
                     if hip.check(name, v, t, dims, dt)[0] == hip.AXON_OK]
            # A variant that does not serve this shape says so in its manifest
            # (an extent of 0 admits nothing), e.g. attention's split key
            # ranges above 16384 query rows.
            assert legal or any(c.extent == 0 for c in cons), (name, v)
            for t in legal:
                why = rejection_reason(spec.tile_args, t, cons)
                if name in SPLITK_BOX:
                    assert why is None or " > extent " in why, (name, v, t, why)
                else:
                    assert why is None, (name, v, t, why)
            if name in SPLITK_BOX and legal:
                assert rejection_reason(spec.tile_args, (1, 1, 1), cons) is None, (name, v)


@pytest.mark.parametrize(
    ("name", "dims", "best"),
    [
        ("matmul_std002", [1024, 512, 16384], (2, 2, 8)),
        ("rmsnorm_matmul_eps", [1024, 512, 16384], (2, 2, 8)),
        # hw variant 3 counts N in units of 256 columns: its fastest is 128 x 512.
        ("qkv_cte", [16384, 512, 8192], {0: (4, 4, 16), 1: (4, 4, 16), 2: (4, 4, 16), 3: (2, 2, 16)}),
    ],
)
def test_default_budget_benches_the_fastest_tuple(name, dims, best):
    """The reference's default flow (manifest filter, then select_diverse with
    a budget of 8 per hw variant, src/axon/bench_runner.py:613-621) benches
    the tuple that a full sweep of every legal tuple of every hw variant
    measured fastest on MI355X at these shapes. Over the uncapped box the
    budget reaches only its corners (1x1x32 at 57.5 us against 2x2x8 at
    34.2 us for the 1024x512x16384 matmul)."""
    from axon.candidate_filter import rejection_reason, select_diverse
    from enzyme_amd.kernel_spec import SEED

    spec = load_spec(name)
    for v in range(hip.variant_count(name)):
        cons = hip.manifest(name, v, dims, hip.AXON_BF16)
        legal = [t for t in product(spec.tile_options, repeat=len(spec.tile_args))
                 if rejection_reason(spec.tile_args, t, cons) is None]
        want = best[v] if isinstance(best, dict) else best
        assert want in select_diverse(legal, budget=8, seed=SEED), (name, v, legal)


def test_manifest_admits_only_legal_tiles():
    """Every tile tuple a variant's manifest admits, at every case in
    eval/sizes.json, is one the library accepts: the candidate filter reads
    only the manifest (src/axon/candidate_filter.py:90-103), so a tuple it
    admits but the library refuses would spend the bench budget on
    "compile: assert" rows."""
    import json

    from axon.candidate_filter import rejection_reason
    from enzyme_amd.dtypes import to_torch
    from tests._specs import spec_inputs

    cases = json.loads((REPO / "eval" / "sizes.json").read_text())
    checked = 0
    for name, per_case in cases.items():
        if name.startswith("_"):
            continue
        spec = load_spec(name)
        for cid, case in per_case.items():
            if cid.startswith("_"):
                continue
            dims = dict(zip(spec.dim_vars, case["sizes"]))
            small = tuple(min(v, 8) for v in case["sizes"])
            _, _, ins = spec_inputs(name, small, dtype=case.get("dtype"))
            codes = [hip.dtype_code(to_torch(a)) for a in ins]
            dvals = [dims[d] for d in spec.dim_vars]
            served = 0
            for v in range(hip.variant_count(name)):
                cons = hip.manifest(name, v, dvals, codes[0])
                tuples = list(product(spec.tile_options, repeat=len(spec.tile_args)))
                admitted = [t for t in tuples if rejection_reason(spec.tile_args, t, cons) is None]
                if not admitted:
                    # A variant without an instantiation for this dtype or
                    # shape admits nothing, and the library agrees.
                    assert all(hip.check(name, v, t, dvals, codes)[0] in (hip.AXON_EDTYPE, hip.AXON_EINVAL)
                               for t in tuples), (name, cid, v)
                    continue
                served += 1
                for t in admitted:
                    st, why = hip.check(name, v, t, dvals, codes)
                    assert st == hip.AXON_OK, (name, cid, v, t, why)
                checked += len(admitted)
            assert served, (name, cid)
    assert checked > 500


@pytest.mark.parametrize(("name", "dims"), [("matmul", [4096, 4096, 4096]), ("matmul_std002", [8192, 8192, 1024]),
                                          ("rmsnorm_matmul", [4096, 4096, 4096]),
                                          ("rmsnorm_matmul_eps", [8192, 8192, 1024])])
def test_manifest_admits_only_legal_tiles_at_large_outputs(name, dims):
    """Shapes whose occupancy box reaches 256 x 256 tiles: the 8-wave hw
    variant (up to 256 x 128) must still admit only tuples it accepts."""
    from axon.candidate_filter import rejection_reason

    spec = load_spec(name)
    codes = [hip.AXON_BF16] * len(spec.input_specs)
    for v in range(hip.variant_count(name)):
        cons = hip.manifest(name, v, dims, codes[0])
        for t in product(spec.tile_options, repeat=len(spec.tile_args)):
            if rejection_reason(spec.tile_args, t, cons) is None:
                st, why = hip.check(name, v, t, dims, codes)
                assert st == hip.AXON_OK, (name, v, t, why)


# Small legal dims per spec; the first dim is set to 0 below.
_EMPTY_DIMS = {"attention_causal": [1, 2, 64, 128], "attention_nkilib": [64, 128],
               "rope_llama3": [1, 64, 4, 2, 128], "rope": [64, 128]}


def test_empty_leading_dimension_is_a_no_op():
    """Every family, every hw variant, both launch entry points: with the
    leading dim 0 every output is empty, and the launch returns AXON_OK
    before touching any pointer, stream or workspace (so null pointers and no
    workspace are accepted and nothing reaches the GPU)."""
    import ctypes

    from enzyme_amd.dtypes import to_torch
    from tests._specs import spec_inputs

    names = sorted(p.name for p in KERNELS.iterdir() if (p / "__init__.py").exists())
    checked = 0
    for name in names:
        spec = load_spec(name)
        _, _, ins = spec_inputs(name, tuple([8] * len(spec.dim_vars)) if name not in _EMPTY_DIMS
                                else tuple(min(d, 128) if d else 8 for d in _EMPTY_DIMS[name]))
        codes = [hip.dtype_code(to_torch(a)) for a in ins]
        dims = [0] + list(_EMPTY_DIMS.get(name, [64] * len(spec.dim_vars)))[1:]
        for v in range(hip.variant_count(name)):
            tiles = next(t for t in product(spec.tile_options, repeat=len(spec.tile_args))
                         if hip.check(name, v, t, dims, codes)[0] == hip.AXON_OK)
            ct = (ctypes.c_int32 * len(tiles))(*tiles)
            cd = (ctypes.c_int64 * len(dims))(*dims)
            cc = (ctypes.c_int32 * len(codes))(*codes)
            n_in, n_out = len(spec.input_specs), len(hip.outputs(name, dims, codes))
            nulls_in = (ctypes.c_void_p * n_in)()
            nulls_out = (ctypes.c_void_p * n_out)()
            rc = hip.lib().axon_variant_launch(name.encode(), v, ct, len(tiles), cd, len(dims), cc, len(codes),
                                               nulls_in, n_in, nulls_out, n_out, None, 0, None)
            assert rc == hip.AXON_OK, (name, v, tiles, hip.last_error())
            rc = hip.lib().axon_variant_launch_noalloc(name.encode(), v, ct, len(tiles), cd, len(dims), cc,
                                                       len(codes), nulls_in, n_in, nulls_out, n_out, None)
            assert rc == hip.AXON_OK, (name, v, tiles, hip.last_error())
            checked += 1
    assert checked >= len(names)


@pytest.mark.parametrize(
    ("name", "tiles", "dims", "dtype", "legal"),
    [
        ("rmsnorm", (1, 1), [1 << 27, 8], "bf16", False),     # 2^27 workgroups of 64 threads
        ("rmsnorm", (16, 1), [1 << 27, 8], "bf16", False),    # 2^23 of 1024
        ("rmsnorm", (1, 1), [1 << 20, 8], "bf16", True),
        ("matmul", (1, 1, 1), [32768, 32768, 32768], "bf16", False),  # 33.5 M workgroups of 256
        ("matmul", (4, 4, 16), [32768, 32768, 32768], "bf16", True),
        ("cumsum_probs", (16, 1), [1 << 23, 64], "f32", False),      # one 1024-thread workgroup per row
        ("cumsum_probs", (1, 1), [1 << 20, 64], "f32", True),
    ],
)
def test_oversized_grids_are_refused(name, tiles, dims, dtype, legal):
    """A dispatch holds fewer than 2^32 work-items: tile tuples whose grid
    would exceed that at these dims are illegal (the compile worker's
    "assert"), not launched and truncated."""
    code = hip.AXON_BF16 if dtype == "bf16" else hip.AXON_F32
    n_in = len(load_spec(name).input_specs)
    st, why = hip.check(name, 0, tiles, dims, [code] * n_in)
    if legal:
        assert st == hip.AXON_OK, why
    else:
        assert st == hip.AXON_EINVAL and "2^32" in why, (st, why)


def test_compile_worker_plans_legal_and_asserts_illegal(tmp_path):
    spec = load_spec("rmsnorm")
    mod = tmp_path / "rmsnorm__v0_t0.py"
    mod.write_text(variant_module_text(spec, {"m": 2048, "n": 4096}, 0, 0, hip.AXON_BF16))
    art = tmp_path / "__v0_t0_tiles_2_2" / "kernel.plan.json"
    key, path, err = _compile_one_variant(
        (str(mod), "rmsnorm", (2, 2), ((2048, 4096), (0,)), {"TILES_IN_BLOCK_M": 2, "TILES_IN_BLOCK_N": 2},
         str(art), "gfx950", 1))
    assert err is None and path == str(art) and art.is_file()
    import json

    plan = json.loads(art.read_text())
    assert plan["tiles"] == [2, 2] and plan["dims"] == [2048, 4096] and plan["kernel"] == "rmsnorm"
    art2 = tmp_path / "__v0_t0_tiles_2_3" / "kernel.plan.json"
    key, path, err = _compile_one_variant(
        (str(mod), "rmsnorm", (2, 3), ((2048, 4096), (0,)), {"TILES_IN_BLOCK_M": 2, "TILES_IN_BLOCK_N": 3},
         str(art2), "gfx950", 1))
    assert path is None and err == "assert" and not art2.exists()


def test_workspace_sizes():
    assert hip.workspace_bytes("rmsnorm", 0, [1, 2], [2048, 4096], [0]) == 0
    ws = hip.workspace_bytes("cumsum_probs", 1, [8, 1], [64, 128256], [2])
    assert ws == 64 * ((128256 + 2047) // 2048) * 8
    assert hip.workspace_bytes("matmul", 0, [2, 2, 4], [1024, 1024, 1024], [0, 0]) == 0
    assert hip.workspace_bytes("matmul", 0, [2, 2, 8], [1024, 512, 16384], [0, 0]) > 8 * 1024 * 512 * 4


def test_qkv_full_width_variant_tiles_and_workspace():
    """qkv_cte hw variant 3 counts TILES_IN_BLOCK_N in units of 256 columns
    (1 or 2) and rows in units of 64 (1 or 2), takes bf16 only, and needs the
    packed w (k rounded up to 64 x N tiles x BN, bf16) ahead of the split-K
    partials and row sums."""
    m, n, k = 16384, 512, 8192
    bf16 = [hip.AXON_BF16] * 4
    assert hip.check("qkv_cte", 3, (2, 2, 16), [m, n, k], bf16)[0] == hip.AXON_OK
    for tiles in [(2, 4, 16), (4, 2, 16), (2, 8, 16)]:
        st, why = hip.check("qkv_cte", 3, tiles, [m, n, k], bf16)
        assert st == hip.AXON_EINVAL and "TILES_IN_BLOCK_N 1 or 2" in why, (tiles, why)
    assert hip.check("qkv_cte", 3, (2, 2, 16), [m, n, k], [hip.AXON_F32] * 4)[0] == hip.AXON_EDTYPE
    splits = k // (16 * 256)
    packed = k * 512 * 2
    assert hip.workspace_bytes("qkv_cte", 3, (2, 2, 16), [m, n, k], bf16) == (
        packed + splits * m * n * 4 + splits * 1 * m * 4)
    # One K range: no split-K data, only the packed w (here 640 columns -> two
    # 512-column tiles, k = 1000 -> 1024 packed rows).
    assert hip.workspace_bytes("qkv_cte", 3, (2, 2, 4), [96, 640, 1000], bf16) == 1024 * 1024 * 2


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(hip, "_lib", None)
    monkeypatch.setattr(hip, "LIB_PATH", tmp_path / "absent.so")
    with pytest.raises(hip.HipLibraryError, match="missing"):
        hip.lib()
