"""Fused int4 dequant + GEMM layers on the HIP library.

API of the reference's ``layers/fused_int4_linear.py`` (FusedInt4Linear
:958-1246, fused_int4_gemm :388-537, FusedInt4LinearPaddedGroups :761-955,
FusedInt4LinearAnyGroup :639-758). Every forward is one launch of
``oc_int4_gemm`` on torch's current stream.

Layout. All classes share one load-time plan (``oc_int4_plan_groups``):
the packed rows are re-laid into uniform groups of ``group_rows`` (a
multiple of 32) physical rows -- odd group sizes get 32-row slots with zero
rows (the reference's ``_repack_groups_to_32``, :94-124), act-order ``g_idx``
sorts rows by group -- and ``oc_int4_prepare`` writes the weight once into
the tiled device layout the kernels stream: 16-column tiles whose 32-row
steps are 256 contiguous bytes, with the tile's scales and zeros (restored
to their value, so v1 and v2 checkpoints run the same kernels) beside them.
The layer keeps only the tiled tensors (``qweight_tiled``, ``scales_tiled``,
``zeros_tiled``); checkpoint-format tensors given on the CPU are held until
the first device forward prepares them. ``state_dict`` / ``load_state_dict``
and the ``qweight`` / ``scales`` / ``qzeros`` attributes use the reference
modules' buffer layouts, translated to and from the tiled one on the device.
"""
from __future__ import annotations

import collections
import weakref

import torch

from .. import _hip, _profile, kernels


def _unpack_host(qweight: torch.Tensor, rows: int) -> torch.Tensor:
    """int32 [R, N] packed along K -> int32 codes [rows, N] (host, load/save time)."""
    q = qweight.to(torch.int64) & 0xFFFFFFFF
    parts = [(q >> (4 * i)) & 0xF for i in range(8)]
    return torch.stack(parts, dim=1).reshape(-1, q.shape[1])[:rows].to(torch.int32)


def _pack_host(codes: torch.Tensor) -> torch.Tensor:
    """int codes [K, N] -> int32 [ceil(K/8), N] packed along K (host, load/save time)."""
    K, N = codes.shape
    full = torch.zeros(((K + 7) // 8 * 8, N), dtype=torch.int64)
    full[:K] = codes.to(torch.int64) & 0xF
    full = full.reshape(-1, 8, N)
    word = torch.zeros((full.shape[0], N), dtype=torch.int64)
    for i in range(8):
        word |= full[:, i, :] << (4 * i)
    return torch.where(word >= 2**31, word - 2**32, word).to(torch.int32)


class _HipGPTQLinear(torch.nn.Module):
    """Shared state and forward of the packed GPTQ int4 layers.

    Device state is the tiled layout only (non-persistent buffers
    ``qweight_tiled`` / ``scales_tiled`` / ``zeros_tiled`` plus the row maps).
    The module's ``state_dict`` holds the reference module's buffers instead
    -- ``qweight``, ``scales``, ``qzeros`` in the checkpoint formats and in the
    layout the reference class registers (``_STATE_LAYOUT``) -- written from
    the tiled layout by ``oc_int4_export``; ``load_state_dict`` takes the same
    tensors and re-runs ``oc_int4_prepare``. ``.qweight`` / ``.scales`` /
    ``.qzeros`` read back the same tensors.

    ``_STATE_LAYOUT``:
      "kpad256"  FusedInt4Linear: K padded to a multiple of 256 with zero rows,
                 zero scales and zero stored zeros (fused_int4_linear.py:989-1005)
      "physical" FusedInt4LinearPaddedGroups: the 32-row group slots
                 (fused_int4_linear.py:796-803), i.e. the physical row order
      "input"    PackedGPTQLinear / FusedInt4LinearAnyGroup: the checkpoint
                 tensors as given (packed_gptq_linear.py:57-60)
    """

    _STATE_LAYOUT = "input"
    wbits = 4

    def _setup(self, in_features: int, out_features: int, qweight: torch.Tensor,
               scales: torch.Tensor, qzeros: torch.Tensor, bias: torch.Tensor | None,
               groupsize: int, g_idx: torch.Tensor | None, v1: bool, kind: str, wbits: int = 4) -> None:
        self.in_features = int(in_features)
        self.out_features = int(out_features)
        self.groupsize = int(groupsize)
        self.v1 = bool(v1)
        self.wbits = int(wbits)
        self._kind = kind
        per = 32 // self.wbits
        if self.out_features % per != 0:
            raise ValueError(f"out_features must be a multiple of {per}, got {self.out_features}")
        for name in ("qweight_tiled", "scales_tiled", "zeros_tiled", "kmap", "kinv",
                     "_src_qweight", "_src_scales", "_src_qzeros"):
            self.register_buffer(name, None, persistent=False)
        self._weights = None
        self._call = None  # kernels.LayerCall bound to the current tiled weights
        self._configure(g_idx, qweight.device)
        # Row and group counts of the checkpoint tensors as given (the "input"
        # state layout reproduces them).
        self._ckpt_rows = int(qweight.shape[0]) if qweight.dim() == 2 else 0
        self._ckpt_groups = int(scales.shape[0]) if scales.dim() == 2 else 0
        self._set_sources(qweight, scales, qzeros, physical=False)
        if bias is not None:
            self.register_buffer("bias", bias.contiguous())
        else:
            self.bias = None

    def _configure(self, g_idx: torch.Tensor | None, device: torch.device) -> None:
        """Plan the physical rows (``oc_int4_plan_groups``) and keep the row maps."""
        plan = kernels.plan_groups(self.in_features, self.groupsize, g_idx)
        self._plan = plan
        self.k_phys = plan.k_phys
        self.group_rows = plan.group_rows
        self.num_phys_groups = plan.num_groups
        # The kernels read activations through kmap (physical -> input row) and
        # kinv (input -> physical row) only when the rows moved.
        self.kmap, self.kinv = kernels.row_maps(plan, device)
        self._call = None

    def _check_sources(self, qweight, scales, qzeros, physical: bool) -> None:
        if qweight.dtype != torch.int32 or qzeros.dtype != torch.int32:
            raise ValueError("qweight and qzeros must be int32")
        if qweight.dim() != 2 or qweight.shape[1] != self.out_features:
            raise ValueError(f"qweight has shape {tuple(qweight.shape)}, expected [*, {self.out_features}]")
        per = 32 // self.wbits
        rows_expected = (self.k_phys if physical else self.in_features + per - 1) // per
        if qweight.shape[0] < rows_expected:
            raise ValueError(f"qweight K-dim mismatch: got {qweight.shape[0]}, expected {rows_expected}")
        G = self.num_phys_groups
        if scales.dim() != 2 or scales.shape[0] < G or scales.shape[1] != self.out_features:
            raise ValueError(f"scales shape {tuple(scales.shape)} does not cover "
                             f"{G} groups x {self.out_features}")
        if qzeros.dim() != 2 or tuple(qzeros.shape[1:]) != (self.out_features // per,) or qzeros.shape[0] < G:
            raise ValueError(f"qzeros shape {tuple(qzeros.shape)} does not cover "
                             f"{G} groups x {self.out_features // per}")

    def _set_sources(self, qweight, scales, qzeros, *, physical: bool) -> None:
        """Checkpoint tensors (input row order, or ``physical`` row order) to be
        written into the tiled layout: now when on the device, else at the
        first device forward."""
        self._check_sources(qweight, scales, qzeros, physical)
        if scales.dtype not in (torch.float16, torch.bfloat16):
            scales = scales.to(torch.float16)
        self._src_qweight, self._src_scales, self._src_qzeros = qweight, scales, qzeros
        self._src_physical = physical
        self.qweight_tiled = self.scales_tiled = self.zeros_tiled = None
        self._weights = self._call = None
        if qweight.is_cuda:
            self._prepare()

    def _prepare(self) -> kernels.TiledWeights:
        """Write the tiled layout on the layer's device and drop the sources."""
        if self._src_physical:  # rows already in physical order: identity map
            w = kernels.prepare(self._src_qweight, self._src_scales, self._src_qzeros,
                                in_features=self.k_phys, out_features=self.out_features, kmap=None,
                                k_phys=self.k_phys, group_rows=self.group_rows, v1=self.v1, wbits=self.wbits)
        else:
            w = kernels.prepare(self._src_qweight, self._src_scales, self._src_qzeros,
                                in_features=self.in_features, out_features=self.out_features,
                                kmap=self.kmap, k_phys=self.k_phys, group_rows=self.group_rows, v1=self.v1,
                                wbits=self.wbits)
        self.qweight_tiled, self.scales_tiled, self.zeros_tiled = w.qt, w.st, w.zt
        self._src_qweight = self._src_scales = self._src_qzeros = None
        self._weights = w
        return w

    def tiled(self) -> kernels.TiledWeights:
        w = self._weights
        if w is None or w.qt is not self.qweight_tiled or w.st is not self.scales_tiled:
            if self.qweight_tiled is None:
                if not self._src_qweight.is_cuda:
                    raise RuntimeError(
                        f"{type(self).__name__} runs on the HIP device; move the layer there first "
                        f"(its weights are on {self._src_qweight.device})")
                return self._prepare()
            w = kernels.TiledWeights(self.qweight_tiled, self.scales_tiled, self.zeros_tiled,
                                     self.out_features, self.k_phys, self.group_rows, self.wbits)
            self._weights = w
        return w

    # ---- reference module state -------------------------------------------------
    def _state_shape(self) -> tuple[int, int]:
        """(code rows, groups) of the reference buffers of this class."""
        if self._STATE_LAYOUT == "kpad256":
            k_pad = (self.in_features + 255) // 256 * 256
            return k_pad, k_pad // self.groupsize
        if self._STATE_LAYOUT == "physical":
            return self.k_phys, max(self._ckpt_groups, self.num_phys_groups)
        return (max(32 // self.wbits * self._ckpt_rows, self.in_features),
                max(self._ckpt_groups, self.num_phys_groups))

    def checkpoint_tensors(self) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """``(qweight, scales, qzeros)`` as the reference module holds them."""
        rows, groups = self._state_shape()
        if self.qweight_tiled is None and self._src_qweight is not None and not self._src_qweight.is_cuda:
            return self._host_checkpoint(rows, groups)
        w = self.tiled()
        row_src = None
        if self._STATE_LAYOUT == "input" and not self._plan.identity:
            live = self._plan.kmap >= 0
            inv = torch.full((rows,), -1, dtype=torch.int32)
            inv[torch.from_numpy(self._plan.kmap[live]).long()] = torch.from_numpy(
                live.nonzero()[0].astype("int32"))
            row_src = inv.to(w.qt.device)
        return kernels.export_checkpoint(w, row_src=row_src, out_rows=rows, out_groups=groups, v1=self.v1)

    def _host_checkpoint(self, rows: int, groups: int):
        """The same tensors from sources still held on the host (before the
        first device move): integer re-layout only."""
        q, s, z = self._src_qweight, self._src_scales, self._src_qzeros
        N = self.out_features

        def fit(t, n, cols):
            out = torch.zeros((n, cols), dtype=t.dtype)
            m = min(n, t.shape[0])
            out[:m] = t[:m]
            return out

        if self._src_physical or self._STATE_LAYOUT == "input":
            return q, s, z
        if self._STATE_LAYOUT == "physical":
            codes = _unpack_host(q, self.in_features)
            kmap = torch.from_numpy(self._plan.kmap).long()
            phys = torch.zeros((self.k_phys, N), dtype=torch.int32)
            live = kmap >= 0
            phys[live] = codes[kmap[live]]
            return _pack_host(phys), s, z
        # kpad256: zero rows, scales and stored zeros past in_features
        G = (self.in_features + self.groupsize - 1) // self.groupsize
        return (fit(fit(q, (self.in_features + 7) // 8, N), rows // 8, N), fit(fit(s, G, N), groups, N),
                fit(fit(z, G, N // 8), groups, N // 8))

    @property
    def qweight(self) -> torch.Tensor:
        return self.checkpoint_tensors()[0]

    @property
    def scales(self) -> torch.Tensor:
        return self.checkpoint_tensors()[1]

    @property
    def qzeros(self) -> torch.Tensor:
        return self.checkpoint_tensors()[2]

    def _save_to_state_dict(self, destination, prefix, keep_vars):
        q, s, z = self.checkpoint_tensors()
        destination[prefix + "qweight"] = q
        destination[prefix + "scales"] = s
        destination[prefix + "qzeros"] = z
        super()._save_to_state_dict(destination, prefix, keep_vars)

    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys,
                              unexpected_keys, error_msgs):
        keys = [prefix + n for n in ("qweight", "scales", "qzeros")]
        present = [k in state_dict for k in keys]
        if all(present):
            try:
                g_key = prefix + "g_idx"
                g_idx = state_dict.get(g_key) if "g_idx" in self._buffers else None
                self.load_checkpoint(*(state_dict[k] for k in keys), g_idx=g_idx)
            except (ValueError, RuntimeError) as e:
                error_msgs.append(f"{prefix}: {e}")
        elif strict:
            missing_keys.extend(k for k, p in zip(keys, present) if not p)
        super()._load_from_state_dict(state_dict, prefix, local_metadata, strict, missing_keys,
                                      unexpected_keys, error_msgs)
        for k in keys:
            if k in unexpected_keys:
                unexpected_keys.remove(k)

    def load_checkpoint(self, qweight: torch.Tensor, scales: torch.Tensor, qzeros: torch.Tensor,
                        g_idx: torch.Tensor | None = None) -> None:
        """Replace the weights by reference-layout tensors (as ``state_dict``
        holds them) and rebuild the tiled layout on the layer's device."""
        ref = self.qweight_tiled if self.qweight_tiled is not None else self._src_qweight
        device = ref.device
        if g_idx is not None:
            self._configure(g_idx, device)
        physical = self._STATE_LAYOUT == "physical"
        if self._STATE_LAYOUT == "input":
            self._ckpt_rows = int(qweight.shape[0])
            self._ckpt_groups = int(scales.shape[0])
        dt = self.scales_tiled.dtype if self.scales_tiled is not None else self._src_scales.dtype
        self._set_sources(qweight.to(device), scales.to(device=device, dtype=dt), qzeros.to(device),
                          physical=physical)

    # ---- forward ----------------------------------------------------------------

    def _gemm(self, x: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
        orig_dtype = x.dtype
        if orig_dtype == torch.float32:
            # fp32 input is computed in fp16 and returned as fp32
            # (fused_int4_linear.py:415-419, :535-536).
            x = x.to(torch.float16)
        flat = x.dim() == 2 and x.shape[1] == self.in_features  # rows already: no view ops
        a_2d = x if flat else x.reshape(-1, self.in_features)
        if _profile.PROFILE_SHAPES:
            _profile.record(self._kind, a_2d.shape[0], self.in_features, self.out_features)
        call, buf = self._call, self._buffers
        if (call is None or call.qt is not buf.get("qweight_tiled") or call.w.st is not buf.get("scales_tiled")
                or call.mid[1] != call.qt.data_ptr()):
            w = self.tiled()
            call = self._call = kernels.LayerCall(w, self.in_features, self.kmap, self.kinv)
        c = call(a_2d, bias)
        out = c if flat else c.reshape(*x.shape[:-1], self.out_features)
        if orig_dtype == torch.float32:
            out = out.to(torch.float32)
        return out

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        # The reference's fused kernels add the bias buffer as stored, in fp32.
        return self._gemm(x, self.bias)

    def dequantize(self, dtype: torch.dtype = torch.float16) -> torch.Tensor:
        """Dense [out_features, in_features] weight, values as the reference's
        ``dequant_gptq_to_fp`` (exact fp32 product, one rounding to dtype)."""
        return kernels.dequant_tiled(self.tiled(), self.kmap, self.in_features, dtype)

    @torch.no_grad()
    def warmup(self, m_values=(32, 128, 256, 1024, 2250)) -> None:
        """Run one forward per M so workspaces are sized before timing.

        The kernels are compiled ahead of time; there is no JIT to trigger.
        """
        ref = self.qweight_tiled if self.qweight_tiled is not None else self._src_qweight
        device = ref.device
        if device.type != "cuda":
            return
        scales = self.scales_tiled if self.scales_tiled is not None else self._src_scales
        dtype = scales.dtype if scales.dtype in (torch.float16, torch.bfloat16) else torch.float16
        for m in m_values:
            if m <= 0:
                continue
            self.forward(torch.zeros((int(m), self.in_features), dtype=dtype, device=device))
        torch.cuda.synchronize(device)

    def _apply(self, fn, recurse=True):
        # Keep integer buffers int32 across .to(dtype=...) and scales 16-bit
        # (fused_int4_linear.py:1230-1246).
        before = {n: getattr(self, n) for n in ("qweight_tiled", "zeros_tiled", "kmap", "_src_qweight",
                                                "_src_qzeros")}
        kinv_before = self.kinv
        self._call = None
        result = super()._apply(fn, recurse=recurse)
        for name, old in before.items():
            new = getattr(self, name)
            if new is not None and new.dtype != torch.int32:
                setattr(self, name, old.to(new.device))
        if self.kinv is not None and self.kinv.dtype != torch.int16:
            self.kinv = kinv_before.to(self.kinv.device)
        for name in ("scales_tiled", "_src_scales"):
            t = getattr(self, name)
            if t is not None and t.dtype not in (torch.float16, torch.bfloat16):
                setattr(self, name, t.to(torch.float16))
        return result

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"wbits={self.wbits}, groupsize={self.groupsize}, v1={self.v1}, k_phys={self.k_phys}, "
                f"group_rows={self.group_rows}, backend=hip")


class FusedInt4Linear(_HipGPTQLinear):
    """Drop-in int4 GPTQ (groupsize 32) Linear on the HIP fused kernels.

    Constructor and attributes as the reference (fused_int4_linear.py:966-1014);
    ``v1`` (keyword) selects the zero convention of the checkpoint format,
    "gptq" (v1, the reference's only mode) or "gptq_v2". Its state holds the
    reference's K-padded buffers (K rounded up to 256, zero rows/scales/zeros).
    """

    _STATE_LAYOUT = "kpad256"

    def __init__(self, in_features: int, out_features: int, qweight: torch.Tensor,
                 scales: torch.Tensor, qzeros: torch.Tensor, bias: torch.Tensor | None = None,
                 groupsize: int = 32, *, v1: bool = True):
        super().__init__()
        assert groupsize == 32, "FusedInt4Linear supports groupsize=32 only"
        # K of the reference's registered buffers (padded to a multiple of 256)
        self._k_padded = (int(in_features) + 255) // 256 * 256
        self._setup(in_features, out_features, qweight, scales, qzeros, bias, 32, None, v1, "fused")

    @classmethod
    def from_gptq_linear(cls, layer) -> "FusedInt4Linear":
        """Build from a GPTQ Linear (4-bit, groupsize 32), reusing its packed buffers."""
        assert layer.wbits == 4, f"FusedInt4Linear requires wbits=4, got {layer.wbits}"
        assert layer.groupsize == 32, f"FusedInt4Linear requires groupsize=32, got {layer.groupsize}"
        return cls(in_features=layer.in_features, out_features=layer.out_features,
                   qweight=layer.qweight, scales=layer.scales.to(torch.float16),
                   qzeros=layer.qzeros, bias=layer.bias if layer.bias is not None else None,
                   groupsize=32, v1=getattr(layer, "v1", True))


class FusedInt4LinearPaddedGroups(_HipGPTQLinear):
    """Odd groupsize (< 32) GPTQ int4 layer, re-laid into 32-row groups.

    Same constructor checks as the reference (fused_int4_linear.py:770-811);
    its state holds the 32-row-slot qweight the reference registers (:796-803).
    """

    _STATE_LAYOUT = "physical"

    def __init__(self, in_features: int, out_features: int, qweight: torch.Tensor,
                 scales: torch.Tensor, qzeros: torch.Tensor, bias: torch.Tensor | None = None,
                 groupsize: int = 32, *, v1: bool = True):
        super().__init__()
        if groupsize == 32:
            raise ValueError("FusedInt4LinearPaddedGroups is only for odd groupsizes")
        if groupsize <= 0 or groupsize > 32:
            raise ValueError(f"groupsize must be in 1..32, got {groupsize}")
        if in_features % groupsize != 0:
            raise ValueError(f"in_features={in_features} must be divisible by groupsize={groupsize}")
        self.num_groups = int(in_features) // int(groupsize)
        self._setup(in_features, out_features, qweight, scales, qzeros, bias, groupsize, None, v1,
                    "padded")
        self.padded_in_features = self.k_phys


class FusedInt4LinearAnyGroup(_HipGPTQLinear):
    """GPTQ int4 layer of any groupsize (reference: fused_int4_linear.py:639-758)."""

    def __init__(self, in_features: int, out_features: int, qweight: torch.Tensor,
                 scales: torch.Tensor, qzeros: torch.Tensor, bias: torch.Tensor | None = None,
                 groupsize: int = 32, *, v1: bool = True):
        super().__init__()
        self._setup(in_features, out_features, qweight, scales, qzeros, bias, groupsize, None, v1,
                    "any_group")


_TILE_CACHE: "collections.OrderedDict[tuple, tuple]" = collections.OrderedDict()
_TILE_CACHE_MAX = 64


def _functional_tiles(qweight, scales, qzeros, K: int, N: int) -> kernels.TiledWeights:
    """Tiled layout of the functional form's weights, cached per tensor triple.

    The functional API has no load step; the tiled layout is written on the
    first call and reused while the same tensor objects, unmodified (their
    version counters), come back. Entries hold weak references, so a freed
    tensor whose address is reused never hits a stale entry.
    """
    key = (qweight.data_ptr(), scales.data_ptr(), qzeros.data_ptr(), scales.dtype, K, N)
    ver = (qweight._version, scales._version, qzeros._version)
    hit = _TILE_CACHE.get(key)
    if hit is not None:
        refs, v, w = hit
        if refs[0]() is qweight and refs[1]() is scales and refs[2]() is qzeros and v == ver:
            _TILE_CACHE.move_to_end(key)
            return w
        del _TILE_CACHE[key]
    w = kernels.prepare(qweight.contiguous(), scales.contiguous(), qzeros.contiguous(), in_features=K,
                        out_features=N, kmap=None, k_phys=K, group_rows=32, v1=True)
    _TILE_CACHE[key] = ((weakref.ref(qweight), weakref.ref(scales), weakref.ref(qzeros)), ver, w)
    while len(_TILE_CACHE) > _TILE_CACHE_MAX:
        _TILE_CACHE.popitem(last=False)
    return w


def fused_int4_gemm(a: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor,
                    qzeros: torch.Tensor, bias: torch.Tensor | None = None,
                    groupsize: int = 32) -> torch.Tensor:
    """``c = a @ dequantize(qweight) + bias`` (reference: fused_int4_linear.py:388-537).

    Same contract: v1 zeros, groupsize 32, fp16/bf16/fp32 input (fp32 is
    computed in fp16 and returned as fp32), scales cast to the activation type.
    """
    assert groupsize == 32, "fused_int4_gemm currently supports groupsize=32 only"
    assert qweight.dtype == torch.int32
    assert qzeros.dtype == torch.int32
    assert a.dtype in (torch.float16, torch.bfloat16, torch.float32), f"unsupported a.dtype={a.dtype}"
    orig_dtype = a.dtype
    if a.dtype == torch.float32:
        a = a.to(torch.float16)
    if scales.dtype != a.dtype:
        scales = scales.to(a.dtype)
    leading_shape = a.shape[:-1]
    K = a.shape[-1]
    a_2d = a.reshape(-1, K)
    N = scales.shape[1]
    assert qweight.shape == (K // 8, N), (
        f"qweight shape mismatch: expected ({K//8}, {N}), got {tuple(qweight.shape)}")
    assert scales.shape == (K // groupsize, N), (
        f"scales shape mismatch: expected ({K//groupsize}, {N}), got {tuple(scales.shape)}")
    assert qzeros.shape == (K // groupsize, N // 8), (
        f"qzeros shape mismatch: expected ({K//groupsize}, {N//8}), got {tuple(qzeros.shape)}")
    assert N % 8 == 0, f"N must be a multiple of 8 (qzeros packing), got N={N}"
    assert K % 32 == 0, f"K must be a multiple of 32 (groupsize), got K={K}"
    if bias is not None:
        bias = bias.to(a.dtype)
    c = kernels.int4_gemm(a_2d, _functional_tiles(qweight, scales, qzeros, K, N), in_features=K, bias=bias)
    out = c.reshape(*leading_shape, N)
    if orig_dtype == torch.float32:
        out = out.to(torch.float32)
    return out


__all__ = [
    "FusedInt4Linear",
    "FusedInt4LinearAnyGroup",
    "FusedInt4LinearPaddedGroups",
    "fused_int4_gemm",
]
