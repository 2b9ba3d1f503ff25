"""DeepSeek-V4 QEP packed layers (layers/dsv4_packed_linear.py:22-102): uint8
int2/int4 codes along the in-dim, groupwise scales/zeros in either
orientation. Device dequant bit-exact against the oracle and the exact-rational
known answers; the fused GEMM bit-exact through one-hot rows and within the
GEMM tolerance; host-resident experts staged through the pinned-memory copy
stream, with routed-expert batches matching the oracle's per-expert loop."""
import numpy as np
import pytest
import torch

from gpu_helpers import assert_gemm_close, bits16, np32, oracle_bits, say
from oracle import onecomp_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _packed(out_f, in_f, wbits, gs, seed, orient="GN", zero_kind="int"):
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 1 << wbits, (out_f, in_f))
    G = (in_f + gs - 1) // gs if gs > 0 else 1
    s = (np.abs(rng.standard_normal((G, out_f))) * 0.02 + 1e-4).astype(np.float16)
    if zero_kind == "int":
        z = rng.integers(0, 1 << wbits, (G, out_f)).astype(np.float16)
    else:
        z = rng.uniform(-0.5, (1 << wbits) + 0.5, (G, out_f)).astype(np.float16)
    if gs <= 0:
        s, z = s.reshape(out_f), z.reshape(out_f)
    elif orient == "NG":
        s, z = s.T.copy(), z.T.copy()
    return {"qweight_packed": torch.from_numpy(O.dsv4_pack(codes, wbits)), "scales": torch.from_numpy(s),
            "qzeros": torch.from_numpy(z), "wbits": wbits, "groupsize": gs, "in_features": in_f}


def _ref_w(p, dtype):
    return O.dequant_dsv4(p["qweight_packed"].numpy(), p["scales"].float().numpy(), p["qzeros"].float().numpy(),
                          p["wbits"], p["groupsize"], p["in_features"], dtype)


def test_dsv4_dequant_kats_on_device(kats):
    from onecomp_runtime import kernels

    for wb in (2, 4):
        cases = [c for c in kats["dsv4_dequant"] if c["wbits"] == wb]
        per = 8 // wb
        n = len(cases)
        codes = np.zeros((n, per), np.int64)
        codes[:, 0] = [c["q"] for c in cases]
        z = np.array([c["zero_f16_bits"] for c in cases], np.uint16).view(np.float16).reshape(n, 1)
        s = np.array([c["scale_f16_bits"] for c in cases], np.uint16).view(np.float16).reshape(n, 1)
        qw = torch.from_numpy(O.dsv4_pack(codes, wb)).to(DEV)
        for dt, key in ((torch.bfloat16, "bf16_bits"), (torch.float16, "f16_bits")):
            say(f"dsv4 KATs wbits={wb} {dt}")
            out = kernels.dsv4_dequant(qw, torch.from_numpy(s).to(DEV), torch.from_numpy(z).to(DEV), wbits=wb,
                                       groupsize=per, in_features=per, dtype=dt)
            assert np.array_equal(bits16(out)[:, 0], np.array([c[key] for c in cases], np.uint16))


@pytest.mark.parametrize("wbits", [2, 4])
@pytest.mark.parametrize("case", ["gs128_GN", "gs64_NG", "per_row", "frac_zero_f16", "ragged_k"])
def test_dsv4_dequant_and_one_hot_gemm_bit_exact(wbits, case):
    from onecomp_runtime.layers import Dsv4PackedLinear, dequant_dsv4_packed

    out_f, in_f, gs, orient, zk, dt = 136, 1024, 128, "GN", "int", torch.bfloat16
    if case == "gs64_NG":
        gs, orient = 64, "NG"
    elif case == "per_row":
        gs = 0
    elif case == "frac_zero_f16":
        zk, dt, gs = "frac", torch.float16, 32
    elif case == "ragged_k":
        in_f, gs = 1000, 100  # not fused: device dequant + F.linear
    p = _packed(out_f, in_f, wbits, gs, seed=wbits * 100 + len(case), orient=orient, zero_kind=zk)
    name = "bf16" if dt == torch.bfloat16 else "f16"
    say(f"dsv4 dequant wbits={wbits} {case}")
    w = dequant_dsv4_packed(p, dtype=dt, device=DEV)
    assert np.array_equal(bits16(w), oracle_bits(_ref_w(p, name), dt))
    mod = Dsv4PackedLinear(p, buffer_device=DEV)
    fused = mod._fused_ok(torch.zeros(1, dtype=dt))
    assert fused == (case != "ragged_k")
    for M in (1, 3, 40, 300):  # M <= 4: the row GEMV; larger: the tiled kernel
        ks = np.random.default_rng(M).integers(0, in_f, M)
        x = torch.zeros((M, in_f), dtype=dt)
        x[torch.arange(M), torch.from_numpy(ks)] = 1.0
        say(f"dsv4 one-hot wbits={wbits} {case} M={M}")
        assert np.array_equal(bits16(mod(x.to(DEV))), oracle_bits(_ref_w(p, name)[:, ks].T, dt))


@pytest.mark.parametrize("wbits", [2, 4])
def test_dsv4_gemm_matches_oracle_with_bias(wbits):
    from onecomp_runtime.layers import Dsv4PackedLinear

    p = _packed(2048, 7168, wbits, 128, seed=20450 + wbits)
    bias = torch.randn(2048, generator=torch.Generator().manual_seed(wbits))
    mod = Dsv4PackedLinear(p, bias=bias, buffer_device=DEV)
    for M in (1, 2, 4, 8, 512):
        x = torch.randn(M, 7168, generator=torch.Generator().manual_seed(M)).to(torch.bfloat16)
        say(f"dsv4 gemm wbits={wbits} M={M} K=7168 N=2048")
        ref = O.linear(np32(x), _ref_w(p, "bf16"), O.round_to(bias.numpy(), "bf16"), "bf16")
        assert_gemm_close(mod(x.to(DEV)), ref, f"dsv4 int{wbits} M={M}")
    xf = torch.randn(3, 7168, generator=torch.Generator().manual_seed(9))
    say("dsv4 fp32 activations")
    out = mod(xf.to(DEV))
    assert out.dtype == torch.float32
    assert_gemm_close(out, O.linear(xf.numpy(), _ref_w(p, "f32"), bias.numpy(), "f32"), "dsv4 fp32")


def test_dsv4_offloaded_experts_match_oracle():
    """Routed experts held in pinned host memory: staged per call through the
    copy stream (prefetch ahead), repeated experts served from their slot."""
    from onecomp_runtime import offload
    from onecomp_runtime.layers import Dsv4PackedLinear, run_routed_experts

    E, K, N, T, topk = 12, 1024, 512, 48, 2
    packs = [_packed(N, K, 2, 128, seed=20460 + e) for e in range(E)]
    experts = [Dsv4PackedLinear(p, buffer_device="cpu") for p in packs]
    assert all(m.qweight_packed.is_pinned() for m in experts)
    g = torch.Generator().manual_seed(20470)
    ids = torch.topk(torch.randn(T, E, generator=g), topk, dim=-1).indices
    x = torch.randn(T, K, generator=g).to(torch.bfloat16)
    before = offload.stager.stats(0)
    say("dsv4 routed experts from host memory")
    y = run_routed_experts(experts, x.to(DEV), ids)
    torch.cuda.synchronize()
    wds = {e: _ref_w(packs[e], "bf16") for e in np.unique(ids.numpy())}
    ref = O.moe(np32(x), ids.numpy(), wds, "bf16")
    assert_gemm_close(y, ref, "offloaded experts")
    # the same batch again: bit-identical; the last experts still in their slots
    y2 = run_routed_experts(experts, x.to(DEV), ids)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    after = offload.stager.stats(0)
    used = len(np.unique(ids.numpy()))
    assert after["copies"] - before["copies"] <= 2 * used
    assert after["hits"] > before["hits"]
    # a host expert called directly equals its device-resident twin
    dev_twin = Dsv4PackedLinear(packs[0], buffer_device=DEV)
    assert torch.equal(experts[0](x.to(DEV)), dev_twin(x.to(DEV)))
    assert torch.equal(experts[0].weight, dev_twin.weight)
