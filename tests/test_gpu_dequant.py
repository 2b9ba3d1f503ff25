"""Bit-exact parity of the HIP unpack/dequant kernels with the oracle
(quant_utils.dequant_gptq_to_fp / dequant_extra_u8_to_weight semantics)."""
import numpy as np
import pytest
import torch

from gpu_helpers import bits16, layer_oracle_inputs, oracle_bits, say
from oracle import onecomp_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.mark.parametrize("K,N,gs,v1,act,out_dtype,scale_dtype", [
    (4096, 4096, 32, True, False, torch.bfloat16, torch.float16),   # gptq_gs32_m16 weights
    (4096, 4096, 32, True, False, torch.float16, torch.float16),
    (3072, 3072, 32, False, False, torch.bfloat16, torch.float16),  # dit_large_m (v2)
    (5120, 1024, 32, True, True, torch.bfloat16, torch.float16),    # act-order g_idx (decode shapes)
    (5120, 5120, 32, True, True, torch.bfloat16, torch.float16),
    (5120, 17408, 32, True, True, torch.bfloat16, torch.float16),
    (17408, 5120, 32, True, True, torch.bfloat16, torch.float16),
    (3072, 12288, 32, False, False, torch.bfloat16, torch.float16),  # the other DiT shapes (v2)
    (12288, 3072, 32, False, False, torch.bfloat16, torch.float16),
    (1040, 3072, 26, True, False, torch.bfloat16, torch.float16),   # odd groups
    (1000, 64, 32, True, False, torch.bfloat16, torch.bfloat16),    # ragged K, bf16 scales
    (256, 64, 128, False, False, torch.float32, torch.float16),
    (1024, 256, 32, True, True, torch.float16, torch.float32),     # fp32 scales: product rounded to fp32 first
    (1024, 256, 32, True, False, torch.bfloat16, torch.float32),
])
def test_gptq_dequant_bit_exact(K, N, gs, v1, act, out_dtype, scale_dtype):
    from onecomp_runtime import quant_utils, synthetic

    say(f"gptq dequant K={K} N={N} gs={gs} v1={v1} act={act} out={out_dtype} scales={scale_dtype}")
    layer = synthetic.gptq_layer(K, N, seed=11, groupsize=gs, v1=v1, act_order=act,
                                 scale_dtype=scale_dtype)
    qw, sc, qz, g_idx = layer_oracle_inputs(layer)
    ref = O.dequant_gptq(qw, sc, qz, g_idx, K, N, {torch.bfloat16: "bf16", torch.float16: "f16",
                                                   torch.float32: "f32"}[out_dtype], v1)
    g = torch.from_numpy(g_idx).to(DEV)
    out = quant_utils.dequant_gptq_to_fp(layer.qweight.to(DEV), layer.scales.to(DEV),
                                         layer.qzeros.to(DEV), g, K, N, out_dtype, v1=v1)
    if out_dtype == torch.float32:
        assert np.array_equal(out.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    else:
        assert np.array_equal(bits16(out), oracle_bits(ref, out_dtype))


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16])
def test_fast_dequant_path_bit_exact(out_dtype):
    """groupsize path without g_idx: the kernel shares dequant8() with the GEMMs."""
    from onecomp_runtime import kernels, synthetic

    K, N = 2048, 512
    say(f"fast dequant {out_dtype}")
    layer = synthetic.gptq_layer(K, N, seed=12)
    qw, sc, qz, g_idx = layer_oracle_inputs(layer)
    ref = O.dequant_gptq(qw, sc, qz, g_idx, K, N, "bf16" if out_dtype == torch.bfloat16 else "f16")
    out = kernels.int4_dequant(layer.qweight.to(DEV), layer.scales.to(DEV), layer.qzeros.to(DEV),
                               None, K, N, out_dtype, v1=True, groupsize=32)
    assert np.array_equal(bits16(out), oracle_bits(ref, out_dtype))


def test_dequant_kats_on_device(kats):
    """The exact-rational known answers, through the device kernel."""
    from onecomp_runtime import kernels

    cases = kats["gptq_dequant"]
    n = len(cases)
    N = (n + 7) // 8 * 8
    codes = np.zeros((8, N), np.int64)
    zeros = np.zeros((1, N), np.int64)
    scales = np.zeros((1, N), np.uint16)
    for i, c in enumerate(cases):
        codes[0, i], zeros[0, i], scales[0, i] = c["w"], c["z"], c["scale_f16_bits"]
    qw = torch.from_numpy(O.pack_rows(codes)).to(DEV)
    qz = torch.from_numpy(O.pack_zeros(zeros, v1=False)).to(DEV)
    sc = torch.from_numpy(scales.view(np.int16)).view(torch.float16).to(DEV)
    for dt, key in ((torch.bfloat16, "bf16_bits"), (torch.float16, "f16_bits")):
        say(f"dequant KATs {dt}")
        out = kernels.int4_dequant(qw, sc, qz, None, 8, N, dt, v1=False, groupsize=32)
        got = bits16(out)[:n, 0]
        assert np.array_equal(got, np.array([c[key] for c in cases], np.uint16))


def test_dequant_8bit_matches_oracle():
    from onecomp_runtime import quant_utils

    rng = np.random.default_rng(5)
    K, N, gs = 256, 32, 64
    codes = rng.integers(0, 256, (K, N))
    zeros = rng.integers(0, 256, (K // gs, N))
    scales = (np.abs(rng.standard_normal((K // gs, N))) * 0.01 + 1e-3).astype(np.float16)
    qw = O.pack_rows(codes, wbits=8)
    qz = O.pack_zeros(zeros, v1=True, wbits=8)
    ref = O.dequant_gptq(qw, scales.astype(np.float32), qz, O.default_g_idx(K, gs), K, N, "bf16",
                         v1=True, wbits=8)
    say("dequant 8-bit")
    out = quant_utils.dequant_gptq_to_fp(torch.from_numpy(qw).to(DEV), torch.from_numpy(scales).to(DEV),
                                         torch.from_numpy(qz).to(DEV),
                                         torch.arange(K, device=DEV) // gs, K, N, torch.bfloat16,
                                         v1=True, wbits=8)
    assert np.array_equal(bits16(out), oracle_bits(ref, torch.bfloat16))


@pytest.mark.parametrize("wbits", [4, 8])
def test_unpack_rows_matches_oracle(wbits):
    from onecomp_runtime import quant_utils

    rng = np.random.default_rng(6)
    packed = rng.integers(-2**31, 2**31, (33, 24), dtype=np.int64).astype(np.int32)
    packed[0, :3] = [np.int32(-2**31), -1, 0x76543210]
    num_rows = 33 * (32 // wbits) - 5
    say(f"unpack rows wbits={wbits}")
    out = quant_utils._unpack_rows(torch.from_numpy(packed).to(DEV), num_rows, wbits)
    assert np.array_equal(out.cpu().numpy(), O.unpack_rows(packed, num_rows, wbits))
    w = quant_utils.unpack_int_weights(torch.from_numpy(packed).to(DEV), wbits, (24, num_rows))
    assert np.array_equal(w.cpu().numpy(), O.unpack_int_weights(packed, wbits, (24, num_rows)))
    qz = packed[:, :3].copy()
    z = quant_utils.unpack_zeros(torch.from_numpy(qz).to(DEV), wbits, 3 * (32 // wbits))
    assert np.array_equal(z.cpu().numpy(), O.unpack_zeros(qz, wbits, 3 * (32 // wbits)))


def _untile(w, N):
    """Tiled tensors -> physical packed rows [K_phys/8, N], scales [G, N], zeros [G, N]."""
    qt, st, zt = w.qt.cpu().numpy(), w.st.cpu(), w.zt.cpu().numpy()
    tiles, KS = qt.shape[:2]
    packed = qt.transpose(1, 3, 0, 2).reshape(KS * 4, tiles * 16)[:, :N]
    G = st.shape[1]
    scales = st.permute(1, 0, 2).reshape(G, tiles * 16)[:, :N]
    zw = zt.view(np.uint32)  # [tiles, G, 2]
    nib = (zw[..., None] >> (4 * np.arange(8, dtype=np.uint32))) & 15  # [tiles, G, 2, 8]
    zeros = nib.reshape(tiles, G, 16).transpose(1, 0, 2).reshape(G, tiles * 16)[:, :N]
    return packed, scales, zeros.astype(np.int32)


def test_prepare_layout_odd_groups():
    """gs 26: the physical rows of the tiled layout are the reference's
    ``_repack_groups_to_32`` output; scales copied, v1 zeros restored (+1)."""
    from onecomp_runtime import kernels, synthetic

    K, N = 1040, 72  # 5 tiles, the last one half full
    layer = synthetic.gptq_layer(K, N, seed=7, groupsize=26)
    plan = kernels.plan_groups(K, 26)
    say("prepare layout gs=26")
    w = kernels.prepare(layer.qweight.to(DEV), layer.scales.to(DEV), layer.qzeros.to(DEV), in_features=K,
                        out_features=N, kmap=torch.from_numpy(plan.kmap).to(DEV), k_phys=plan.k_phys,
                        group_rows=plan.group_rows, v1=True)
    assert w.qt.shape == (5, plan.k_phys // 32, 16, 4) and w.zt.shape == (5, K // 26, 2)
    packed, scales, zeros = _untile(w, N)
    ref_pad, kp = O.repack_groups_to_32(layer.qweight.numpy(), K, N, 26)
    assert kp == plan.k_phys and np.array_equal(packed, ref_pad)
    assert torch.equal(scales, layer.scales)
    assert np.array_equal(zeros, (O.unpack_zeros(layer.qzeros.numpy(), 4, N) + 1) & 15)
    # columns beyond N in the last tile are zero
    assert not w.qt[-1, :, 8:].any() and not w.st[-1, :, 8:].any() and not w.zt[-1, :, 1].any()


def test_prepare_layout_act_order_v2():
    """act-order: physical row r holds input row kmap[r] (rows sorted by group)."""
    from onecomp_runtime import kernels, synthetic

    K, N = 1024, 48
    layer = synthetic.gptq_layer(K, N, seed=9, groupsize=128, v1=False, act_order=True)
    plan = kernels.plan_groups(K, 128, layer.g_idx)
    say("prepare layout act-order v2")
    w = kernels.prepare(layer.qweight.to(DEV), layer.scales.to(DEV), layer.qzeros.to(DEV), in_features=K,
                        out_features=N, kmap=torch.from_numpy(plan.kmap).to(DEV), k_phys=plan.k_phys,
                        group_rows=plan.group_rows, v1=False)
    packed, scales, zeros = _untile(w, N)
    assert np.array_equal(O.unpack_rows(packed, K, 4), layer.codes.numpy()[plan.kmap])
    assert torch.equal(scales, layer.scales)
    assert np.array_equal(zeros, O.unpack_zeros(layer.qzeros.numpy(), 4, N))


@pytest.mark.parametrize("K,N,gs,v1,act,out_dtype,scale_dtype", [
    (1040, 72, 26, True, False, torch.bfloat16, torch.float16),     # odd groups, ragged tile
    (5120, 1024, 32, True, True, torch.bfloat16, torch.float16),    # act-order gs 32
    (1024, 256, 128, False, True, torch.float16, torch.bfloat16),   # act-order gs 128, v2
    (1000, 40, 32, True, False, torch.float32, torch.float16),      # ragged K and N
    (4096, 512, 32, True, False, torch.float16, torch.float16),
])
def test_dequant_tiled_bit_exact(K, N, gs, v1, act, out_dtype, scale_dtype):
    """prepare -> dequant_tiled reproduces dequant_gptq_to_fp bit for bit."""
    from onecomp_runtime import kernels, synthetic

    say(f"dequant tiled K={K} N={N} gs={gs} v1={v1} act={act} out={out_dtype} scales={scale_dtype}")
    layer = synthetic.gptq_layer(K, N, seed=13, groupsize=gs, v1=v1, act_order=act, scale_dtype=scale_dtype)
    qw, sc, qz, g_idx = layer_oracle_inputs(layer)
    ref = O.dequant_gptq(qw, sc, qz, g_idx, K, N, {torch.bfloat16: "bf16", torch.float16: "f16",
                                                   torch.float32: "f32"}[out_dtype], v1)
    plan = kernels.plan_groups(K, gs, layer.g_idx if act else None)
    kmap = None if plan.identity else torch.from_numpy(plan.kmap).to(DEV)
    w = kernels.prepare(layer.qweight.to(DEV), layer.scales.to(DEV), layer.qzeros.to(DEV), in_features=K,
                        out_features=N, kmap=kmap, k_phys=plan.k_phys, group_rows=plan.group_rows, v1=v1)
    out = kernels.dequant_tiled(w, kmap, K, out_dtype)
    assert out.shape == (N, K)
    if out_dtype == torch.float32:
        assert np.array_equal(out.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    else:
        assert np.array_equal(bits16(out), oracle_bits(ref, out_dtype))


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("G", [1, 8])
def test_rtn_dequant_bit_exact(out_dtype, G):
    from onecomp_runtime import quant_utils

    rng = np.random.default_rng(8)
    rows, K = 96, 256
    q = rng.integers(0, 256, (rows, K // 2)).astype(np.uint8)
    s = (np.abs(rng.standard_normal((rows, G))) * 0.05 + 1e-3).astype(np.float16)
    z = rng.uniform(-3, 18, (rows, G)).astype(np.float16)  # non-integer zeros: per-op rounding matters
    name = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}[out_dtype]
    ref = O.rtn_dequant(q, s.astype(np.float32), z.astype(np.float32), K, rows, name)
    say(f"rtn dequant {out_dtype} G={G}")
    out = quant_utils.dequant_extra_u8_to_weight(torch.from_numpy(q).to(DEV), torch.from_numpy(s).to(DEV),
                                                 torch.from_numpy(z).to(DEV), K, rows, out_dtype)
    assert np.array_equal(out.float().cpu().numpy(), ref)


def test_rtn_kats_on_device(kats):
    from onecomp_runtime import quant_utils

    cases = kats["rtn_dequant"]
    n = len(cases)
    q = torch.tensor([[c["w"]] for c in cases], dtype=torch.uint8, device=DEV)
    s = torch.tensor([[c["scale_f16_bits"]] for c in cases], dtype=torch.int32).to(torch.int16).view(torch.float16).to(DEV)
    z = torch.tensor([[c["zero_f16_bits"]] for c in cases], dtype=torch.int32).to(torch.int16).view(torch.float16).to(DEV)
    for dt, key in ((torch.bfloat16, "bf16_bits"), (torch.float16, "f16_bits")):
        say(f"rtn KATs {dt}")
        out = quant_utils.dequant_extra_u8_to_weight(q, s, z, 1, n, dt)
        assert np.array_equal(bits16(out)[:, 0], np.array([c[key] for c in cases], np.uint16))
