"""Host-resident weights streamed to the device on demand (DSV4 routed experts).

The reference keeps offloaded experts' packed buffers on the CPU and moves
them to the GPU inside every forward (layers/dsv4_packed_linear.py:32-33,
:94-96): a synchronous copy from pageable memory per call. Here:

  * the host copies live in pinned memory, so a copy is one DMA that runs
    asynchronously beside the compute;
  * copies go out on a side stream of default priority into a small pool of
    device slots per device; the compute stream waits for a slot's copy event
    before the kernel reads it, and the next copy into that slot waits for the
    kernel's event, so ``prefetch`` of the next experts overlaps the current
    expert's GEMM;
  * a slot remembers whose weights it holds (identity and version of the host
    tensors): an expert routed again while its slot is intact is not copied
    again (least recently used slot is replaced).

Each staged item is a list of host tensors; their device copies are laid out
in one slot buffer at 256-byte aligned offsets.
"""
from __future__ import annotations

import threading
from dataclasses import dataclass, field

import torch

_ALIGN = 256


def _align(n: int) -> int:
    return (n + _ALIGN - 1) // _ALIGN * _ALIGN


@dataclass
class _Slot:
    buf: torch.Tensor | None = None
    key: tuple | None = None  # identity + versions of the host tensors held
    views: list | None = None
    copied: torch.cuda.Event | None = None  # the copy into the slot has landed
    released: torch.cuda.Event | None = None  # the last reader of the slot is done
    stamp: int = 0
    pending: bool = False  # prefetched, not yet read: not evicted while others can be


@dataclass
class _DevicePool:
    stream: torch.cuda.Stream
    slots: list = field(default_factory=list)
    clock: int = 0
    copies: int = 0
    hits: int = 0


class DeviceStager:
    """Pool of device slots fed from pinned host tensors (one pool per device)."""

    def __init__(self, num_slots: int = 4) -> None:
        self.num_slots = int(num_slots)
        self._pools: dict[int, _DevicePool] = {}
        self._lock = threading.Lock()

    def _pool(self, device: torch.device) -> _DevicePool:
        idx = device.index if device.index is not None else torch.cuda.current_device()
        pool = self._pools.get(idx)
        if pool is None:
            with torch.cuda.device(idx):
                pool = _DevicePool(torch.cuda.Stream(device=idx))
                pool.slots = [_Slot() for _ in range(self.num_slots)]
            self._pools[idx] = pool
        return pool

    @staticmethod
    def _key(tensors) -> tuple:
        return tuple((id(t), t.data_ptr(), t._version, t.numel(), t.dtype) for t in tensors)

    def stage(self, tensors: list[torch.Tensor], device: torch.device,
              prefetch: bool = False) -> tuple[list[torch.Tensor], _Slot]:
        """Device copies of ``tensors`` (pinned host tensors) in a slot; the
        copy is enqueued on the pool's copy stream. Call ``use`` before reading
        them on a compute stream and ``release`` after the last read. A
        ``prefetch`` keeps its slot from eviction until a later call reads it;
        the slot replaced is the least recently used of the others."""
        with self._lock:
            pool = self._pool(device)
            pool.clock += 1
            key = self._key(tensors)
            for slot in pool.slots:
                if slot.key == key:
                    slot.stamp = pool.clock
                    slot.pending = slot.pending and prefetch
                    pool.hits += 1
                    return slot.views, slot
            free = [s for s in pool.slots if not s.pending] or pool.slots
            slot = min(free, key=lambda s: s.stamp)
            slot.stamp = pool.clock
            slot.pending = prefetch
            sizes = [_align(t.numel() * t.element_size()) for t in tensors]
            need = sum(sizes)
            if slot.buf is None or slot.buf.numel() < need:
                with torch.cuda.device(device):
                    if slot.released is not None:
                        torch.cuda.current_stream().wait_event(slot.released)
                    slot.buf = torch.empty(need, dtype=torch.uint8, device=device)
            views, off = [], 0
            for t, n in zip(tensors, sizes):
                nbytes = t.numel() * t.element_size()
                views.append(slot.buf[off:off + nbytes].view(t.dtype).view(t.shape))
                off += n
            with torch.cuda.stream(pool.stream):
                if slot.released is not None:
                    pool.stream.wait_event(slot.released)  # its previous reader is done
                for v, t in zip(views, tensors):
                    v.copy_(t, non_blocking=True)
                slot.copied = torch.cuda.Event()
                slot.copied.record(pool.stream)
            slot.buf.record_stream(pool.stream)
            slot.key, slot.views = key, views
            pool.copies += 1
            return views, slot

    @staticmethod
    def use(slot: _Slot) -> None:
        """The current stream waits for the slot's copy."""
        if slot.copied is not None:
            torch.cuda.current_stream().wait_event(slot.copied)

    @staticmethod
    def release(slot: _Slot) -> None:
        """The slot may be overwritten once the current stream's work so far is done."""
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream())
        slot.released = ev

    def stats(self, device: torch.device | int = 0) -> dict:
        idx = device if isinstance(device, int) else (device.index or 0)
        pool = self._pools.get(idx)
        return {"copies": pool.copies, "hits": pool.hits} if pool else {"copies": 0, "hits": 0}


stager = DeviceStager()


def pinned(t: torch.Tensor) -> torch.Tensor:
    """A pinned host copy of ``t`` (allocated pinned; existing memory is never registered)."""
    if t.device.type == "cpu" and t.is_pinned():
        return t.contiguous()
    if not torch.cuda.is_available():  # no device to pin for: a plain host copy
        return t.detach().to("cpu").contiguous()
    out = torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
    out.copy_(t)
    return out
