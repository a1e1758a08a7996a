"""LoRA overlay on the device.

Mirrors the reference's adapter classes (paths under /root/reference/lora/src/
main/java/cab/ml/juno/lora/):

* ``LoraAdapter``     LoraAdapter (LoraAdapter.java:35-98): rank, inDim, outDim,
                      scale = alpha / rank, A [rank][inDim], B [outDim][rank];
                      ``forward(x)`` = (B (A x)) * scale.  The matrices live in HBM
                      and ``apply_dev`` adds the delta to a projection's output on
                      the device for a batch of rows (jh_lora_apply_dev).
* ``LoraAdapterSet``  LoraAdapterSet (LoraAdapterSet.java:34-140): adapters keyed
                      "layer:proj", ``get`` / ``add``, and the reference's checkpoint
                      format (``save`` / ``load``: big-endian, magic "LORA", version 1).

The decoders apply the adapters for "wq" and "wv" right after the Q and V
projections (LoraTrainableHandler.java:475-476).  Training (backward, gradients)
is not on this path.
"""
from __future__ import annotations

import ctypes
import struct

import numpy as np

from . import _lib
from .matvec import IllegalArgumentException, IOException, _check

_MAGIC, _VERSION = 0x4C4F5241, 1


def _torch():
    import torch  # device memory and streams: plumbing around the HIP library
    return torch


class LoraAdapter:
    """A rank-r adapter; its matrices move to HBM on first device use."""

    def __init__(self, rank: int, in_dim: int, out_dim: int, alpha: float, a, b, device: int = 0):
        if rank < 1:
            raise IllegalArgumentException("rank must be >= 1")
        if in_dim < 1:
            raise IllegalArgumentException("inDim must be >= 1")
        if out_dim < 1:
            raise IllegalArgumentException("outDim must be >= 1")
        a = np.ascontiguousarray(a, dtype=np.float32).reshape(-1)
        b = np.ascontiguousarray(b, dtype=np.float32).reshape(-1)
        if a.size != rank * in_dim or b.size != out_dim * rank:
            raise IllegalArgumentException(
                f"a.length={a.size} (want {rank * in_dim}) or b.length={b.size} (want {out_dim * rank}) mismatch")
        self.rank, self.in_dim, self.out_dim = rank, in_dim, out_dim
        self.scale = float(np.float32(alpha) / np.float32(rank))  # Java float alpha / int rank
        self.a_host, self.b_host = a.copy(), b.copy()
        self.device = device
        self._dev = None  # (A, B) in HBM, uploaded on first device use

    def _device_mats(self):
        if self._dev is None:
            torch = _torch()
            dev = torch.device("cuda", self.device)
            self._dev = (torch.from_numpy(self.a_host).to(dev), torch.from_numpy(self.b_host).to(dev))
        return self._dev

    @classmethod
    def from_weights(cls, rank: int, in_dim: int, out_dim: int, alpha: float, a, b) -> "LoraAdapter":
        """LoraAdapter.fromWeights (LoraAdapter.java:72-77)."""
        return cls(rank, in_dim, out_dim, alpha, a, b)

    @property
    def alpha(self) -> float:
        return float(np.float32(self.scale) * np.float32(self.rank))

    def apply_dev(self, d_x: int, d_y: int, batch: int = 1, stream=None) -> None:
        """y[b] += (B (A x[b])) * scale for b < batch (device pointers, [batch][dim])."""
        torch = _torch()
        a, b = self._device_mats()
        s = ctypes.c_void_p((stream or torch.cuda.current_stream()).cuda_stream)
        _check(_lib.load().jh_lora_apply_dev(ctypes.c_void_p(a.data_ptr()), ctypes.c_void_p(b.data_ptr()),
                                         self.rank, self.in_dim, self.out_dim, self.scale, ctypes.c_void_p(d_x),
                                         batch, ctypes.c_void_p(d_y), s))

    def forward(self, x) -> np.ndarray:
        """LoraAdapter.forward (LoraAdapter.java:79-98) for one host vector."""
        torch = _torch()
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        if x.size != self.in_dim:
            raise IllegalArgumentException(f"x.length={x.size} != inDim={self.in_dim}")
        dev = self._device_mats()[0].device
        dx = torch.from_numpy(x).to(dev)
        dy = torch.zeros(self.out_dim, device=dev)
        self.apply_dev(dx.data_ptr(), dy.data_ptr(), 1)
        torch.cuda.synchronize()
        return dy.cpu().numpy()


class LoraAdapterSet:
    """Adapters keyed "layer:proj" (LoraAdapterSet.java:39-61)."""

    def __init__(self):
        self._adapters: dict = {}

    @staticmethod
    def key(layer: int, proj: str) -> str:
        return f"{layer}:{proj}"

    def add(self, layer: int, proj: str, adapter: LoraAdapter) -> None:
        self._adapters[self.key(layer, proj)] = adapter

    def get(self, layer: int, proj: str):
        return self._adapters.get(self.key(layer, proj))

    def size(self) -> int:
        return len(self._adapters)

    def as_map(self) -> dict:
        return dict(self._adapters)

    def save(self, path) -> None:
        """The reference's checkpoint layout (LoraAdapterSet.java:68-89)."""
        with open(path, "wb") as f:
            f.write(struct.pack(">iii", _MAGIC, _VERSION, len(self._adapters)))
            for key, a in self._adapters.items():
                kb = key.encode("utf-8")
                f.write(struct.pack(">i", len(kb)) + kb)
                f.write(struct.pack(">iiif", a.rank, a.in_dim, a.out_dim, a.alpha))
                f.write(a.a_host.astype(">f4").tobytes())
                f.write(a.b_host.astype(">f4").tobytes())

    @classmethod
    def load(cls, path) -> "LoraAdapterSet":
        """LoraAdapterSet.load (LoraAdapterSet.java:91-124); each adapter moves to HBM on first use."""
        s = cls()
        with open(path, "rb") as f:
            data = f.read()
        pos = 0

        def take(n):
            nonlocal pos
            if pos + n > len(data):
                raise IOException("truncated LoRA checkpoint")
            out = data[pos:pos + n]
            pos += n
            return out

        magic, version, count = struct.unpack(">iii", take(12))
        if magic != _MAGIC:
            raise IOException(f"Not a LoRA checkpoint (magic=0x{magic & 0xFFFFFFFF:x})")
        if version != _VERSION:
            raise IOException(f"Unsupported LoRA checkpoint version: {version}")
        for _ in range(count):
            (klen,) = struct.unpack(">i", take(4))
            key = take(klen).decode("utf-8")
            rank, in_dim, out_dim, alpha = struct.unpack(">iiif", take(16))
            a = np.frombuffer(take(4 * rank * in_dim), dtype=">f4").astype(np.float32)
            b = np.frombuffer(take(4 * out_dim * rank), dtype=">f4").astype(np.float32)
            s._adapters[key] = LoraAdapter.from_weights(rank, in_dim, out_dim, alpha, a, b)
        return s
