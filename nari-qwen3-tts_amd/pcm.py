"""PCM16 of the codec's waveform and its device-to-host handoff.

``pcm16`` replaces CodecExecutor._pcm16 (executor/codec.py:236-238): clamp to [-1, 1], scale by
32767, round half to even, int16, in one HIP launch (``nq_codec_pcm16``) with no float copy of the
clamped waveform.

``PcmTransferPool`` keeps the engine-facing interface of the reference's transfer pool
(executor/pcm.py:55-143: ``prepare(capacity)``, ``begin(source) -> transfer``, ``transfer.poll()``
returning the bytes once the copy landed, ``discard_when_ready`` / ``discard_if_ready``,
``available`` / ``active``) over one pinned int16 arena cut into ``capacity`` equal lanes: a transfer
leases a lane index, its copy runs on the pool's own default-priority stream behind the producer's
work, and the lane returns to the free set when the bytes are taken or the transfer is discarded.
"""

from __future__ import annotations

import torch

from . import _lib


def pcm16(wav: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """int16 PCM of a float32 device waveform (any shape): round(clamp(wav, -1, 1) * 32767)."""

    if wav.dtype != torch.float32:
        raise TypeError("codec waveform must be float32")
    _lib.require_device(wav)
    src = wav if wav.is_contiguous() else wav.contiguous()
    if out is None:
        out = torch.empty(src.shape, dtype=torch.int16, device=src.device)
    elif out.dtype != torch.int16 or out.shape != src.shape or not out.is_contiguous() or out.device != src.device:
        raise ValueError("out must be a contiguous int16 tensor of the waveform's shape on its device")
    _lib.call("nq_codec_pcm16", src.data_ptr(), src.numel(), None, out.data_ptr(), _lib.stream(src.device))
    return out


class PcmTransfer:
    """One device-to-host copy of PCM into a leased lane of the pool's pinned arena."""

    __slots__ = ("source", "samples", "event", "pool", "lane", "payload")

    def __init__(self, source: torch.Tensor, samples: int, event, pool: "PcmTransferPool", lane: int) -> None:
        self.source = source
        self.samples = samples
        self.event = event
        self.pool = pool
        self.lane: int | None = lane
        self.payload: bytes | None = None

    def poll(self) -> bytes | None:
        """The PCM bytes once the copy has landed (the lane is then free again), else None."""

        if self.payload is None:
            if not self.event.query():
                return None
            if self.lane is None:
                raise RuntimeError("ready PCM transfer lost its host storage")
            self.payload = self.pool._lane_bytes(self.lane, self.samples)
            self.pool._free_lane(self.lane)
            self.lane = None
        return self.payload

    def discard_when_ready(self) -> None:
        if self.payload is None and self.lane is not None:
            self.event.synchronize()
            self.pool._free_lane(self.lane)
            self.lane = None

    def discard_if_ready(self) -> bool:
        """Free a cancelled transfer's lane without waiting; False while its copy is in flight."""

        if self.payload is not None or self.lane is None:
            return True
        if not self.event.query():
            return False
        self.pool._free_lane(self.lane)
        self.lane = None
        return True


class PcmTransferPool:
    def __init__(self, *, maximum_samples: int, device: torch.device | None) -> None:
        if isinstance(maximum_samples, bool) or not isinstance(maximum_samples, int):
            raise TypeError("PCM host capacity must be an integer")
        if maximum_samples < 0:
            raise ValueError("PCM host capacity must be non-negative")
        self.maximum_samples = maximum_samples
        self.device = None if device is None else torch.device(device)
        self._arena = torch.empty(0, dtype=torch.int16, pin_memory=True)
        self._free: list[int] = []
        self._lanes = 0
        self._stream: torch.cuda.Stream | None = None

    @property
    def available(self) -> int:
        return len(self._free)

    @property
    def active(self) -> int:
        return self._lanes - len(self._free)

    def prepare(self, capacity: int) -> None:
        """Hold at least ``capacity`` lanes of ``maximum_samples`` (grown only while nothing is in flight)."""

        if isinstance(capacity, bool) or not isinstance(capacity, int):
            raise TypeError("PCM transfer capacity must be an integer")
        if capacity < 1:
            raise ValueError("PCM transfer capacity must be positive")
        if self.maximum_samples < 1 or capacity <= self._lanes:
            return
        if self.active:
            raise RuntimeError("PCM transfer pool cannot grow while copies are active")
        self._arena = torch.empty(capacity * self.maximum_samples, dtype=torch.int16, pin_memory=True)
        self._lanes = capacity
        self._free = list(range(capacity - 1, -1, -1))
        if self.device is not None and self._stream is None:
            self._stream = torch.cuda.Stream(device=self.device)

    def _lane_bytes(self, lane: int, samples: int) -> bytes:
        at = lane * self.maximum_samples
        return self._arena[at: at + samples].numpy().tobytes()

    def _free_lane(self, lane: int) -> None:
        if lane in self._free or not 0 <= lane < self._lanes:
            raise RuntimeError("PCM transfer pool release underflow")
        self._free.append(lane)

    def begin(self, source: torch.Tensor) -> PcmTransfer:
        """Queue the copy of ``source`` (device int16, any shape) behind the current stream's work."""

        if not isinstance(source, torch.Tensor) or not source.is_cuda:
            raise TypeError("PCM transfer source must be a CUDA tensor")
        if source.dtype is not torch.int16:
            raise TypeError("Codec PCM must use torch.int16")
        flat = source.detach().contiguous().reshape(-1)
        samples = flat.numel()
        if samples > self.maximum_samples:
            raise RuntimeError("Codec PCM exceeds the preallocated transfer capacity")
        if not self._free:
            raise RuntimeError("PCM transfer pool is exhausted")
        lane = self._free.pop()
        if self._stream is None:
            self._stream = torch.cuda.Stream(device=source.device)
        at = lane * self.maximum_samples
        self._stream.wait_stream(torch.cuda.current_stream(source.device))
        with torch.cuda.stream(self._stream):
            self._arena[at: at + samples].copy_(flat, non_blocking=True)
            flat.record_stream(self._stream)
            event = torch.cuda.Event()
            event.record(self._stream)
        return PcmTransfer(flat, samples, event, self, lane)


__all__ = ["PcmTransfer", "PcmTransferPool", "pcm16"]
