"""Reference module state: ``state_dict`` / ``load_state_dict`` / ``.qweight``
in the buffer layouts the reference's modules register, and the loader's
contract. CPU tests cover layers still holding host tensors (the layout code
on the host); the ``gpu`` tests cover the device export (``oc_int4_export``)
and reloading reference-format state into device layers, checked against the
oracle."""
import json

import numpy as np
import pytest
import torch

from gpu_helpers import assert_gemm_close, layer_oracle_inputs, np32, say
from oracle import onecomp_oracle as O

DEV = "cuda:0"


def _kpad_reference_state(layer, K: int, N: int):
    """The reference FusedInt4Linear buffers (fused_int4_linear.py:989-1045):
    K padded to a multiple of 256, zero rows / scales / stored zeros."""
    k_pad = (K + 255) // 256 * 256
    qw = np.zeros((k_pad // 8, N), np.int32)
    qw[: K // 8] = layer.qweight.numpy()[: K // 8]
    sc = np.zeros((k_pad // 32, N), np.float16)
    sc[: K // 32] = layer.scales.numpy()
    qz = np.zeros((k_pad // 32, N // 8), np.int32)
    qz[: K // 32] = layer.qzeros.numpy()
    return qw, sc, qz


def _padded_reference_state(layer, K: int, N: int, gs: int):
    """The reference FusedInt4LinearPaddedGroups buffers (:796-803)."""
    qw, kp = O.repack_groups_to_32(layer.qweight.numpy(), K, N, gs)
    return qw, layer.scales.numpy(), layer.qzeros.numpy(), kp


def _assert_state(sd, prefix, qw, sc, qz):
    assert np.array_equal(sd[prefix + "qweight"].cpu().numpy(), qw)
    assert np.array_equal(sd[prefix + "scales"].cpu().float().numpy(), np.asarray(sc, np.float32))
    assert np.array_equal(sd[prefix + "qzeros"].cpu().numpy(), qz)


# -- host-held layers (CPU) ---------------------------------------------------
@pytest.mark.parametrize("K", [1024, 1056])
def test_fused_state_is_kpadded_on_host(K):
    from onecomp_runtime import FusedInt4Linear, synthetic

    N = 64
    layer = synthetic.gptq_layer(K, N, seed=7)
    mod = FusedInt4Linear(K, N, layer.qweight, layer.scales, layer.qzeros)
    sd = mod.state_dict()
    assert list(sd) == ["qweight", "scales", "qzeros"]
    _assert_state(sd, "", *_kpad_reference_state(layer, K, N))
    assert mod._k_padded == (K + 255) // 256 * 256
    assert np.array_equal(mod.qweight.numpy(), sd["qweight"].numpy())


def test_padded_groups_state_is_32_row_slots_on_host():
    from onecomp_runtime import synthetic
    from onecomp_runtime.layers import FusedInt4LinearPaddedGroups

    K, N, gs = 1040, 64, 26
    layer = synthetic.gptq_layer(K, N, seed=8, groupsize=gs, pad_rows_to=1056)
    mod = FusedInt4LinearPaddedGroups(K, N, layer.qweight, layer.scales, layer.qzeros, groupsize=gs)
    qw, sc, qz, kp = _padded_reference_state(layer, K, N, gs)
    assert mod.padded_in_features == kp == 1280
    _assert_state(mod.state_dict(), "", qw, sc, qz)


def test_packed_state_is_verbatim_with_g_idx_on_host():
    from onecomp_runtime import PackedGPTQLinear, synthetic

    K, N = 512, 64
    layer = synthetic.gptq_layer(K, N, seed=9, act_order=True)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(1))
    mod = PackedGPTQLinear(K, N, layer.qweight, layer.scales, layer.qzeros, g_idx=layer.g_idx, bias=bias,
                           groupsize=32)
    sd = mod.state_dict()
    assert list(sd) == ["qweight", "scales", "qzeros", "g_idx", "bias"]
    _assert_state(sd, "", layer.qweight.numpy(), layer.scales.numpy(), layer.qzeros.numpy())
    assert np.array_equal(sd["g_idx"].numpy(), layer.g_idx.numpy())


def test_load_state_dict_on_host_replans_act_order():
    """A new g_idx in the loaded state re-plans the physical rows."""
    from onecomp_runtime import PackedGPTQLinear, synthetic

    K, N = 256, 32
    a = synthetic.gptq_layer(K, N, seed=10, act_order=True)
    b = synthetic.gptq_layer(K, N, seed=11, act_order=True)
    mod = PackedGPTQLinear(K, N, a.qweight, a.scales, a.qzeros, g_idx=a.g_idx, groupsize=32)
    src = PackedGPTQLinear(K, N, b.qweight, b.scales, b.qzeros, g_idx=b.g_idx, groupsize=32)
    res = mod.load_state_dict(src.state_dict())
    assert not res.missing_keys and not res.unexpected_keys
    assert np.array_equal(mod.g_idx.numpy(), b.g_idx.numpy())
    order = np.argsort(b.g_idx.numpy(), kind="stable")
    assert np.array_equal(mod._plan.kmap, order.astype(np.int32))
    _assert_state(mod.state_dict(), "", b.qweight.numpy(), b.scales.numpy(), b.qzeros.numpy())


def test_load_state_dict_reports_missing_and_bad_shapes():
    from onecomp_runtime import FusedInt4Linear, synthetic

    layer = synthetic.gptq_layer(256, 32, seed=12)
    mod = FusedInt4Linear(256, 32, layer.qweight, layer.scales, layer.qzeros)
    with pytest.raises(RuntimeError, match="Missing key"):
        mod.load_state_dict({"qweight": layer.qweight})
    with pytest.raises(RuntimeError, match="qweight"):
        mod.load_state_dict({"qweight": layer.qweight[:4], "scales": layer.scales, "qzeros": layer.qzeros})
    res = mod.load_state_dict({"qweight": layer.qweight}, strict=False)
    assert "scales" in res.missing_keys


class _TinyBlock(torch.nn.Module):
    def __init__(self, cfg):
        super().__init__()
        d, h = cfg["dim"], cfg["hidden"]
        self.norm = torch.nn.LayerNorm(d)
        self.up = torch.nn.Linear(d, h)
        self.mid = torch.nn.Linear(h, h, bias=False)
        self.down = torch.nn.Linear(h, d, bias=False)
        self.register_buffer("step", torch.zeros(1, dtype=torch.int64))

    def forward(self, x):
        x = torch.nn.functional.gelu(self.up(self.norm(x)))
        return self.down(torch.nn.functional.gelu(self.mid(x)))


def _write_tiny_checkpoint(path, d=256, h=416, fmt="gptq", extra=None, seed_offset=0):
    """gs32 (up), odd gs 26 (mid), act-order (down) layers in one checkpoint."""
    from safetensors.torch import save_file

    from onecomp_runtime import synthetic

    v1 = fmt == "gptq"
    so = seed_offset
    up = synthetic.gptq_layer(d, h, seed=100 + so, v1=v1)
    mid = synthetic.gptq_layer(h, h, seed=101 + so, groupsize=26, v1=v1)
    down = synthetic.gptq_layer(h, d, seed=102 + so, act_order=True, v1=v1)
    gen = torch.Generator().manual_seed(5 + so)
    bias = torch.randn(h, generator=gen).to(torch.float16)
    tensors = {
        "norm.weight": torch.rand(d, generator=gen) + 0.5, "norm.bias": torch.randn(d, generator=gen) * 0.1,
        "step": torch.tensor([3]),
        "up.qweight": up.qweight, "up.scales": up.scales, "up.qzeros": up.qzeros, "up.bias": bias,
        "mid.qweight": mid.qweight, "mid.scales": mid.scales, "mid.qzeros": mid.qzeros,
        "down.qweight": down.qweight, "down.scales": down.scales, "down.qzeros": down.qzeros,
        "down.g_idx": down.g_idx.to(torch.int32),
    }
    tensors.update(extra or {})
    layers = [dict(name="up", wbits=4, groupsize=32, actorder=False, in_features=d, out_features=h),
              dict(name="mid", wbits=4, groupsize=26, actorder=False, in_features=h, out_features=h),
              dict(name="down", wbits=4, groupsize=32, actorder=True, in_features=h, out_features=d)]
    meta = {"config_json": json.dumps({"dim": d, "hidden": h, "_private": 1}),
            "quant_layers_json": json.dumps(layers), "checkpoint_format": fmt}
    save_file(tensors, str(path), metadata=meta)
    return dict(up=up, mid=mid, down=down, bias=bias, tensors=tensors, meta=meta, d=d, h=h)


def test_loader_contract_on_host(tmp_path, capsys):
    from onecomp_runtime import load_int4_model

    path = tmp_path / "tiny.safetensors"
    ck = _write_tiny_checkpoint(path)
    seen_cfg = {}

    def build(cfg):
        seen_cfg.update(cfg)
        return _TinyBlock(cfg)

    model = load_int4_model(str(path), build, device="cpu", backend="auto", label="t")
    assert seen_cfg == {"dim": 256, "hidden": 416}
    assert [type(getattr(model, n)).__name__ for n in ("up", "mid", "down")] == [
        "FusedInt4Linear", "FusedInt4LinearPaddedGroups", "PackedGPTQLinear"]
    rep = model.onecomp_load_report
    assert rep.kinds["hip"] == 3 and rep.tensors == 3 and rep.quant_layers == ["up", "mid", "down"]
    assert "[t] 3 quantized layers (hip=3)" in capsys.readouterr().out
    assert not model.training and int(model.step) == 3
    sd = model.state_dict()
    up, mid, down, d, h = ck["up"], ck["mid"], ck["down"], ck["d"], ck["h"]
    _assert_state(sd, "up.", *_kpad_reference_state(up, d, h))
    qw, sc, qz, _ = _padded_reference_state(mid, h, h, 26)
    _assert_state(sd, "mid.", qw, sc, qz)
    _assert_state(sd, "down.", down.qweight.numpy(), down.scales.numpy(), down.qzeros.numpy())
    assert np.array_equal(sd["down.g_idx"].numpy(), down.g_idx.numpy())
    assert torch.equal(sd["up.bias"], ck["bias"])
    assert torch.equal(sd["norm.weight"], ck["tensors"]["norm.weight"].to(torch.bfloat16))


def test_loader_errors_on_host(tmp_path):
    from safetensors.torch import save_file

    from onecomp_runtime import load_int4_model

    bare = tmp_path / "bare.safetensors"
    save_file({"w": torch.zeros(2)}, str(bare))
    with pytest.raises(ValueError, match="metadata"):
        load_int4_model(str(bare), _TinyBlock, device="cpu")
    extra = tmp_path / "extra.safetensors"
    _write_tiny_checkpoint(extra, extra={"stray.weight": torch.zeros(3)})
    with pytest.raises(RuntimeError, match="unexpected keys"):
        load_int4_model(str(extra), _TinyBlock, device="cpu")
    # a filtered tensor the model needs is missing
    ok = tmp_path / "ok.safetensors"
    _write_tiny_checkpoint(ok)
    with pytest.raises(RuntimeError, match="missing keys"):
        load_int4_model(str(ok), _TinyBlock, device="cpu", tensor_filter=lambda k: k != "norm.bias")
    # the model lacks a quant layer's parent module
    from onecomp_runtime import synthetic

    nested = tmp_path / "nested.safetensors"
    lay = synthetic.gptq_layer(64, 32, seed=13)
    save_file({"blk.proj.qweight": lay.qweight, "blk.proj.scales": lay.scales, "blk.proj.qzeros": lay.qzeros},
              str(nested), metadata={"config_json": "{}", "quant_layers_json": json.dumps(
                  [dict(name="blk.proj", wbits=4, groupsize=32, actorder=False, in_features=64,
                        out_features=32)])})
    with pytest.raises(KeyError):
        load_int4_model(str(nested), lambda cfg: torch.nn.Sequential(), device="cpu")
    # a quant layer filtered out keeps its meta Linear: meta leftover
    with pytest.raises(RuntimeError, match="meta"):
        load_int4_model(str(ok), _TinyBlock, device="cpu", quant_layer_filter=lambda n: n != "mid")
    with pytest.raises(ValueError):
        load_int4_model(str(ok), _TinyBlock, device="cpu", backend="nope")
    with pytest.raises(RuntimeError, match="gemlite"):
        load_int4_model(str(ok), _TinyBlock, device="cpu", backend="gemlite")


# -- device layers (GPU) --------------------------------------------------------
@pytest.mark.gpu
@pytest.mark.parametrize("case", ["gs32_k1024", "gs32_k1056_v2", "gs26", "actorder", "gs128", "anygroup"])
def test_device_state_dict_matches_reference_layout(case):
    """oc_int4_export writes back exactly the reference module's buffers."""
    from onecomp_runtime import FusedInt4Linear, PackedGPTQLinear, synthetic
    from onecomp_runtime.layers import FusedInt4LinearAnyGroup, FusedInt4LinearPaddedGroups

    N = 96
    say(f"device state_dict {case}")
    if case.startswith("gs32"):
        K = 1056 if "1056" in case else 1024
        v1 = "v2" not in case
        layer = synthetic.gptq_layer(K, N, seed=20, v1=v1)
        mod = FusedInt4Linear(K, N, layer.qweight.to(DEV), layer.scales.to(DEV), layer.qzeros.to(DEV), v1=v1)
        expect = _kpad_reference_state(layer, K, N)
    elif case == "gs26":
        K = 520
        layer = synthetic.gptq_layer(K, N, seed=21, groupsize=26)
        mod = FusedInt4LinearPaddedGroups(K, N, layer.qweight.to(DEV), layer.scales.to(DEV),
                                          layer.qzeros.to(DEV), groupsize=26)
        expect = _padded_reference_state(layer, K, N, 26)[:3]
    elif case == "anygroup":
        K = 576
        layer = synthetic.gptq_layer(K, N, seed=22, groupsize=64)
        mod = FusedInt4LinearAnyGroup(K, N, layer.qweight.to(DEV), layer.scales.to(DEV), layer.qzeros.to(DEV),
                                      groupsize=64)
        expect = (layer.qweight.numpy(), layer.scales.numpy(), layer.qzeros.numpy())
    else:
        K, gs = 1024, (128 if case == "gs128" else 32)
        layer = synthetic.gptq_layer(K, N, seed=23, groupsize=gs, act_order=case == "actorder")
        g = layer.g_idx.to(DEV) if layer.g_idx is not None else None
        mod = PackedGPTQLinear(K, N, layer.qweight.to(DEV), layer.scales.to(DEV), layer.qzeros.to(DEV),
                               g_idx=g, groupsize=gs)
        expect = (layer.qweight.numpy(), layer.scales.numpy(), layer.qzeros.numpy())
    sd = mod.state_dict()
    assert sd["qweight"].is_cuda
    _assert_state(sd, "", *expect)


@pytest.mark.gpu
@pytest.mark.parametrize("case", ["gs32_v1", "gs26", "actorder_v2"])
def test_device_load_reference_state_matches_oracle(case):
    """Reference-format (K-padded, v1) state loaded into a device layer that
    held other weights gives the oracle's output for the loaded weights."""
    from onecomp_runtime import FusedInt4Linear, PackedGPTQLinear, synthetic
    from onecomp_runtime.layers import FusedInt4LinearPaddedGroups

    N = 128
    say(f"device load_state_dict {case}")
    if case == "gs32_v1":
        K = 1056
        a = synthetic.gptq_layer(K, N, seed=30)
        b = synthetic.gptq_layer(K, N, seed=31)
        mod = FusedInt4Linear(K, N, a.qweight.to(DEV), a.scales.to(DEV), a.qzeros.to(DEV))
        qw, sc, qz = _kpad_reference_state(b, K, N)
        state = dict(qweight=torch.from_numpy(qw), scales=torch.from_numpy(sc), qzeros=torch.from_numpy(qz))
    elif case == "gs26":
        K = 1040
        a = synthetic.gptq_layer(K, N, seed=32, groupsize=26)
        b = synthetic.gptq_layer(K, N, seed=33, groupsize=26)
        mod = FusedInt4LinearPaddedGroups(K, N, a.qweight.to(DEV), a.scales.to(DEV), a.qzeros.to(DEV),
                                          groupsize=26)
        qw, sc, qz, _ = _padded_reference_state(b, K, N, 26)
        state = dict(qweight=torch.from_numpy(qw), scales=torch.from_numpy(sc), qzeros=torch.from_numpy(qz))
    else:
        K = 1024
        a = synthetic.gptq_layer(K, N, seed=34, act_order=True, v1=False)
        b = synthetic.gptq_layer(K, N, seed=35, act_order=True, v1=False)
        mod = PackedGPTQLinear(K, N, a.qweight.to(DEV), a.scales.to(DEV), a.qzeros.to(DEV),
                               g_idx=a.g_idx.to(DEV), groupsize=32, v1=False)
        state = dict(qweight=b.qweight, scales=b.scales, qzeros=b.qzeros, g_idx=b.g_idx)
    res = mod.load_state_dict(state)
    assert not res.missing_keys and not res.unexpected_keys
    for M in (1, 5, 300):
        x = synthetic.activations(M, K, seed=36 + M)
        ref = O.gptq_linear(np32(x), *layer_oracle_inputs(b), K, N, "bf16", b.v1)
        assert_gemm_close(mod(x.to(DEV)), ref, f"{case} M={M}")
    # and the state reads back as loaded
    sd = mod.state_dict()
    for k in ("qweight", "scales", "qzeros"):
        assert np.array_equal(sd[k].cpu().numpy(), np.asarray(state[k]))


@pytest.mark.gpu
def test_loader_state_round_trip(tmp_path):
    """load -> state_dict -> (safetensors file) -> load_state_dict into a
    model loaded from other weights: the outputs equal the first model's bit
    for bit and match the oracle."""
    from safetensors.torch import load_file, save_file

    from onecomp_runtime import load_int4_model, synthetic

    ck = _write_tiny_checkpoint(tmp_path / "a.safetensors", fmt="gptq")
    say("loader round trip: load A")
    m1 = load_int4_model(str(tmp_path / "a.safetensors"), _TinyBlock, device=DEV, warmup_m_values=(1, 64))
    sd_path = tmp_path / "state.safetensors"
    save_file({k: v.detach().cpu().contiguous() for k, v in m1.state_dict().items()}, str(sd_path))
    # a second checkpoint, same architecture, other weights
    other = _write_tiny_checkpoint(tmp_path / "b.safetensors", fmt="gptq", seed_offset=50)
    say("loader round trip: load B, then A's state")
    m2 = load_int4_model(str(tmp_path / "b.safetensors"), _TinyBlock, device=DEV, warmup=False)
    x = synthetic.activations(9, ck["d"], seed=40).to(DEV)
    with torch.no_grad():
        before = m2(x)
    res = m2.load_state_dict(load_file(str(sd_path)))
    assert not res.missing_keys and not res.unexpected_keys
    with torch.no_grad():
        o1, o2 = m1(x), m2(x)
    assert torch.equal(o1, o2) and not torch.equal(before, o2)
    up, mid, down, d, h = ck["up"], ck["mid"], ck["down"], ck["d"], ck["h"]
    norm_w = ck["tensors"]["norm.weight"].to(torch.bfloat16).float()
    norm_b = ck["tensors"]["norm.bias"].to(torch.bfloat16).float()
    xn = torch.nn.functional.layer_norm(x.float().cpu(), (d,), norm_w, norm_b).to(torch.bfloat16)
    a1 = O.gptq_linear(np32(xn), *layer_oracle_inputs(up), d, h, "bf16", bias=ck["bias"].float().numpy())
    g1 = torch.nn.functional.gelu(torch.from_numpy(a1).to(torch.bfloat16)).float().numpy()
    a2 = O.gptq_linear(g1, *layer_oracle_inputs(mid), h, h, "bf16")
    g2 = torch.nn.functional.gelu(torch.from_numpy(a2).to(torch.bfloat16)).float().numpy()
    ref = O.gptq_linear(g2, *layer_oracle_inputs(down), h, d, "bf16")
    assert_gemm_close(o2, ref, "round trip")
    del other
