"""Host-side checks that need no GPU: the C ABI library loads and exports
every declared symbol, the host-only layout planner, backend routing and
argument errors, and the synthetic data packers."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import onecomp_oracle as O

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "onecomp_hip.h"


def _declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(oc_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    from onecomp_runtime import _hip

    names = _declared_functions()
    assert len(names) >= 12
    lib = ctypes.CDLL(str(_hip.LIB_PATH))
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_hip.SIGNATURES), set(names) ^ set(_hip.SIGNATURES)


def test_layer_call_binding_loads_and_validates():
    """The CPython binding of the per-layer GEMM call is built beside the
    library and rejects bad bindings and calls before reaching the device."""
    from onecomp_runtime import _hip, _occall

    fn = ctypes.cast(_hip.lib().oc_int4_gemm, ctypes.c_void_p).value
    with pytest.raises(ValueError):
        _occall.Layer(0, 4, 64, None, None, 0, None, 16, 64, 32, None, None)  # no entry point
    with pytest.raises(ValueError):
        _occall.Layer(fn, 3, 64, None, None, 0, None, 16, 64, 32, None, None)  # wbits
    h = _occall.Layer(fn, 4, 64, None, None, 0, None, 16, 64, 32, None, None)
    with pytest.raises(TypeError):
        h(0, 64, 1, 1)  # eleven arguments
    with pytest.raises(ValueError):
        h(0, 64, 1, -1, None, 0, 0, 16, None, 0, 0)  # negative M, refused before the call


def test_status_strings_and_version():
    from onecomp_runtime import _hip

    lib = _hip.lib()
    assert lib.oc_status_string(0) == b"OC_OK"
    assert lib.oc_status_string(_hip.OC_ERR_SHAPE) == b"OC_ERR_SHAPE"
    assert lib.oc_version() >= 100


def test_error_mapping_and_last_error():
    from onecomp_runtime import _hip, kernels

    with pytest.raises(ValueError, match="K must be positive"):
        kernels.plan_groups(0, 32)
    assert "K must be positive" in _hip.last_error()
    with pytest.raises(NotImplementedError):
        _hip.check(_hip.OC_ERR_UNSUPPORTED, "x")
    with pytest.raises(RuntimeError):
        _hip.check(_hip.OC_ERR_HIP, "x")


@pytest.mark.parametrize("K,gs", [(4096, 32), (5120, 128), (1040, 26), (1000, 32), (96, 13), (64, 64)])
def test_plan_groups_default_grouping(K, gs):
    from onecomp_runtime import kernels

    p = kernels.plan_groups(K, gs)
    G = -(-K // gs)
    assert p.num_groups == G
    assert p.group_rows % 32 == 0 and p.group_rows >= min(gs, K)
    assert p.k_phys == G * p.group_rows
    valid = p.kmap[p.kmap >= 0]
    assert np.array_equal(np.sort(valid), np.arange(K))  # every column exactly once
    rows = np.nonzero(p.kmap >= 0)[0]
    assert np.array_equal(rows // p.group_rows, p.kmap[rows] // gs)  # row's group == column's group
    assert np.array_equal(p.kmap[p.kinv], np.arange(K))  # kinv: each column's physical row
    assert p.identity == (gs % 32 == 0 and K % gs == 0) or (p.identity and K % 32 == 0)


def test_plan_groups_act_order_sorts_by_group_stably():
    from onecomp_runtime import kernels

    rng = np.random.default_rng(0)
    K, gs = 512, 32
    g_idx = rng.permutation(K) // gs
    p = kernels.plan_groups(K, gs, torch.from_numpy(g_idx))
    assert p.k_phys == K and p.group_rows == 32 and not p.identity
    assert np.array_equal(p.kmap, np.argsort(g_idx, kind="stable"))
    assert np.array_equal(p.kinv[p.kmap], np.arange(p.k_phys))  # kinv inverts kmap
    # identity g_idx is recognised
    p2 = kernels.plan_groups(K, gs, torch.arange(K) // gs)
    assert p2.identity


def test_plan_groups_rejects_bad_g_idx():
    from onecomp_runtime import kernels

    with pytest.raises(ValueError):
        kernels.plan_groups(64, 32, torch.full((64,), -1))
    with pytest.raises(ValueError):
        kernels.plan_groups(64, 32, torch.zeros(10, dtype=torch.long))
    with pytest.raises(NotImplementedError):  # one giant group among many tiny ones
        g = torch.arange(4096) // 1
        g[:4000] = 0
        kernels.plan_groups(4096, 32, g)


def test_synthetic_packers_agree_with_oracle():
    from onecomp_runtime import synthetic

    layer = synthetic.gptq_layer(72, 16, seed=1, groupsize=32, v1=True)
    assert np.array_equal(layer.qweight.numpy(), O.pack_rows(layer.codes.numpy()))
    assert np.array_equal(layer.qzeros.numpy(), O.pack_zeros(layer.zeros.numpy(), v1=True))
    v2 = synthetic.gptq_layer(64, 16, seed=1, v1=False)
    assert np.array_equal(v2.qzeros.numpy(), O.pack_zeros(v2.zeros.numpy(), v1=False))
    padded = synthetic.gptq_layer(1040, 8, seed=2, groupsize=26, pad_rows_to=1056)
    assert padded.qweight.shape == (132, 8) and (padded.qweight[130:] == 0).all()
    rtn = synthetic.rtn_layer(4, 10, seed=3)
    assert np.array_equal(O.rtn_unpack(rtn.qweight_u8.numpy(), 10), rtn.codes.numpy())
    # 8-bit GPTQ and DSV4 generators: the same draws packed by the oracle
    l8 = synthetic.gptq8_layer(256, 64, seed=4, groupsize=128)
    g = torch.Generator().manual_seed(4)
    codes = torch.randint(0, 256, (256, 64), generator=g, dtype=torch.int32)
    zeros = torch.randint(0, 256, (2, 64), generator=g, dtype=torch.int32)
    assert np.array_equal(l8.qweight.numpy(), O.pack_rows(codes.numpy(), 8))
    assert np.array_equal(l8.qzeros.numpy(), O.pack_zeros(zeros.numpy(), True, 8))
    for wb in (2, 4):
        pk = synthetic.dsv4_layer(64, 256, wbits=wb, seed=5)
        g = torch.Generator().manual_seed(5)
        c = torch.randint(0, 1 << wb, (64, 256), generator=g, dtype=torch.int32)
        assert np.array_equal(pk["qweight_packed"].numpy(), O.dsv4_pack(c.numpy(), wb))


def test_resolve_backend_and_dtype():
    from onecomp_runtime import backend

    assert backend.resolve_backend("auto") == "hip"
    assert backend.resolve_backend(None) == "hip"
    assert backend.resolve_backend("fused") == "fused"
    assert backend.resolve_backend("auto", use_fused=False) == "eager"
    with pytest.raises(ValueError):
        backend.resolve_backend("tensorrt")
    for b in ("gemlite", "a8w4", "nvfp4_ffn"):
        with pytest.raises(RuntimeError):
            backend.resolve_backend(b)
    assert backend.resolve_dtype("bf16") is torch.bfloat16
    with pytest.raises(ValueError):
        backend.resolve_dtype("int8")


def test_routing_predicates():
    from onecomp_runtime import backend

    base = dict(wbits=4, groupsize=32, in_features=4096, out_features=4096, actorder=False)
    assert backend.can_use_fused(base)
    assert not backend.can_use_fused({**base, "actorder": True})
    assert backend.can_use_fused_padded_groups({**base, "groupsize": 26, "in_features": 1040})
    assert not backend.can_use_fused_padded_groups(base)
    assert backend.is_v1({}) and backend.is_v1({"checkpoint_format": "gptq"})
    assert not backend.is_v1({"checkpoint_format": "gptq_v2"})


def test_modules_refuse_host_tensors_without_fallback():
    from onecomp_runtime.layers import FusedInt4Linear, FusedInt4LinearPaddedGroups

    layer = O.pack_rows(np.zeros((64, 16), np.int64))
    lin = FusedInt4Linear(64, 16, torch.from_numpy(layer), torch.ones(2, 16, dtype=torch.float16),
                          torch.zeros(2, 2, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="HIP device"):
        lin(torch.zeros(1, 64, dtype=torch.bfloat16))
    with pytest.raises(AssertionError):
        FusedInt4Linear(64, 16, torch.from_numpy(layer), torch.ones(1, 16, dtype=torch.float16),
                        torch.zeros(1, 2, dtype=torch.int32), groupsize=64)
    with pytest.raises(ValueError):
        FusedInt4LinearPaddedGroups(64, 16, torch.from_numpy(layer),
                                    torch.ones(2, 16, dtype=torch.float16),
                                    torch.zeros(2, 2, dtype=torch.int32), groupsize=32)
    # host-built layers keep the checkpoint tensors; the layout is written on the device
    padded = FusedInt4LinearPaddedGroups(52, 16, torch.from_numpy(O.pack_rows(np.zeros((52, 16)))),
                                         torch.ones(2, 16, dtype=torch.float16),
                                         torch.zeros(2, 2, dtype=torch.int32), groupsize=26)
    assert padded.qweight_tiled is None and padded.padded_in_features == 64
    with pytest.raises(RuntimeError, match="HIP device"):
        padded(torch.zeros(1, 52, dtype=torch.bfloat16))


def test_loader_rejects_checkpoint_without_metadata(tmp_path):
    from safetensors.torch import save_file

    from onecomp_runtime import load_int4_model

    path = tmp_path / "plain.safetensors"
    save_file({"w": torch.zeros(2)}, str(path))
    with pytest.raises(ValueError, match="config_json"):
        load_int4_model(str(path), lambda cfg: torch.nn.Linear(2, 2), device="cpu")


def test_planner_takes_stream_mfma_for_small_batches():
    """Batches of 3..16 rows take the balanced-range kernel (its workspace is
    exactly the 512 KB swap-cell area) when their activation rows fit in LDS
    and the workgroup streams at least half as many weight bytes as it stages;
    otherwise the whole-tile MFMA kernel (no workspace, or gathered rows)."""
    from onecomp_runtime import _hip

    f = _hip.lib().oc_int4_gemm_workspace_bytes
    cells = 512 * 1024
    # (M, K_phys, N, has_kmap) -> stream?
    cases = {
        (8, 5120, 5120, 1): True, (8, 5120, 17408, 1): True,
        (4, 5120, 17408, 0): True, (16, 2048, 16400, 0): True,
        (16, 2048, 16384, 0): False,  # 1024 tiles, no gather: whole tiles are even
        (8, 17408, 5120, 1): False,   # 8 rows of K = 17408 exceed LDS: global rows (below)
        (16, 4096, 4096, 0): False,   # 128 KB staged for 32 KB of weights per workgroup
        (17, 1024, 16384, 0): False,  # beyond 16 rows
    }
    for (M, K, N, kmap), stream in cases.items():
        nbytes = f(M, N, K, 32, kmap, 0)
        assert (nbytes == cells) == stream, (M, K, N, kmap, nbytes)
    # Rows beyond LDS on an uneven tile count: the same ranges over rows read
    # from global memory (the counter area, plus act-order rows gathered first).
    assert f(4, 5120, 17408, 32, 0, 0) == cells
    assert f(8, 5120, 17408, 32, 1, 0) == cells + 8 * 17408 * 2
    assert f(16, 4096, 4096, 32, 0, 0) == 0  # 256 tiles: whole tiles are even
    # A narrow layer (64 tiles) runs two workgroups per tile over global rows.
    assert f(8, 1024, 5120, 32, 1, 0) == cells + 8 * 5120 * 2


def test_conv_tile_prepare_rejects_bad_arguments():
    """The tile-layout prepare entry points check pointers, shapes and dtypes
    before they launch anything (no device needed for these calls)."""
    from onecomp_runtime import _hip

    lib = _hip.lib()
    F16, BF16, F32 = _hip.OC_DTYPE_F16, _hip.OC_DTYPE_BF16, _hip.OC_DTYPE_F32
    p = 1 << 12  # a non-NULL, 16-byte aligned stand-in: never dereferenced on these paths
    # oc_rtn_tile_prepare(qweight, N, row_bytes, K, scales, zeros, dtype, G, qt, sz, fast, stream)
    assert lib.oc_rtn_tile_prepare(None, 16, 64, 128, p, p, F16, 4, p, p, p, None) == _hip.OC_ERR_INVALID_ARGUMENT
    assert lib.oc_rtn_tile_prepare(p, 16, 64, 120, p, p, F16, 4, p, p, p, None) == _hip.OC_ERR_SHAPE  # K % 32
    assert lib.oc_rtn_tile_prepare(p, 16, 64, 128, p, p, F16, 8, p, p, p, None) == _hip.OC_ERR_SHAPE  # 16-row groups
    assert lib.oc_rtn_tile_prepare(p, 16, 32, 128, p, p, F16, 4, p, p, p, None) == _hip.OC_ERR_SHAPE  # short rows
    assert lib.oc_rtn_tile_prepare(p, 16, 64, 128, p, p, F32, 4, p, p, p, None) == _hip.OC_ERR_INVALID_ARGUMENT
    assert "16-bit" in _hip.last_error()
    # oc_rtn_tile_prepare_t(qweight, K, row_bytes, N, scales, zeros, scale_dtype, G, x_dtype, qt, szt, fast, stream)
    assert lib.oc_rtn_tile_prepare_t(p, 64, 64, 128, p, p, F16, 4, BF16, None, p, p, None) == \
        _hip.OC_ERR_INVALID_ARGUMENT
    assert lib.oc_rtn_tile_prepare_t(p, 48, 64, 128, p, p, F16, 4, BF16, p, p, p, None) == _hip.OC_ERR_SHAPE  # K
    assert lib.oc_rtn_tile_prepare_t(p, 64, 64, 128, p, p, F16, 16, BF16, p, p, p, None) == _hip.OC_ERR_SHAPE  # gs 8
    assert lib.oc_rtn_tile_prepare_t(p, 64, 64, 128, p, p, F16, 4, F32, p, p, p, None) == \
        _hip.OC_ERR_INVALID_ARGUMENT
