"""InferencePipeline with a real forwardBatch, on the device.

Mirrors the reference's pipeline contract (paths under
/root/reference/node/src/main/java/cab/ml/juno/node/):

* ``forward(request_id, tokens, start_pos)``  InferencePipeline.forward
  (InferencePipeline.java:36-45): the last token of ``tokens`` at position
  ``start_pos`` (getInitialActivation, LlamaTransformerHandler.java:651-660),
  against the KV cache of ``request_id`` (:670-679)
* ``forward_batch(request_ids, all_tokens, start_positions)``
  InferencePipeline.forwardBatch (:47-69): the reference's default is a serial
  loop over forward(); here the N requests are stacked and every layer runs
  once for all of them (batched GEMVs, [q, k, v] grouped: the B <= 2 GEMV
  kernels, fp16 MFMA from B = 3, one launch per group; [gate, up] and SwiGLU in
  one launch; one batched rope + KV-append + attention launch pair)
* ``vocab_size()``  InferencePipeline.vocabSize (:71-75)
* ``evict(request_id)``  LlamaTransformerHandler.evict (:496-504)
* ``lora``  an optional LoraAdapterSet whose "wq" / "wv" adapters are added after
  the Q and V projections (LoraTrainableHandler.java:475-476)

KV caches are one slot per live request in [layers][slots][max_seq][kv_dim]
HBM arrays; a slot is zeroed when a request takes it (the reference allocates
a fresh zeroed array per new requestId, :675-676).  There is no host path.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from .decode import LlamaWeights
from .matvec import IllegalArgumentException, IllegalStateException, _check

_V = ctypes.c_void_p


def _torch():
    import torch  # device memory and streams: plumbing around the HIP library
    return torch


class LlamaBatchPipeline:
    """A node holding every layer, the embeddings and the output projection."""

    def __init__(self, weights: LlamaWeights, max_seq: int, max_batch: int = 64, max_requests: int | None = None,
                 device: int = 0, lora=None):
        torch = _torch()
        if weights.token_embd is None:
            raise IllegalStateException("token input needs token_embd.weight on the device")
        if max_batch < 1 or max_batch > 4096:
            raise IllegalArgumentException(f"max_batch={max_batch} outside [1, 4096]")
        self.w, self.cfg, self.max_seq, self.max_batch = weights, weights.cfg, max_seq, max_batch
        self.lora = lora  # LoraAdapterSet: "wq" / "wv" deltas after the Q and V projections
        self.n_slots = max_requests or max_batch
        c = self.cfg
        self.L = _lib.load()
        dev = torch.device("cuda", device)
        f32 = dict(device=dev, dtype=torch.float32)
        B = max_batch
        self.k_cache = torch.zeros(c.num_layers, self.n_slots, max_seq, c.kv_dim, **f32)
        self.v_cache = torch.zeros(c.num_layers, self.n_slots, max_seq, c.kv_dim, **f32)
        self.x = torch.zeros(B, c.hidden_dim, **f32)
        self.xn = torch.zeros(B, c.hidden_dim, **f32)
        self.q = torch.zeros(B, c.hidden_dim, **f32)
        self.k = torch.zeros(B, c.kv_dim, **f32)
        self.v = torch.zeros(B, c.kv_dim, **f32)
        self.att = torch.zeros(B, c.hidden_dim, **f32)
        self.proj = torch.zeros(B, c.hidden_dim, **f32)
        self.gate = torch.zeros(B, c.intermediate_size, **f32)
        self.up = torch.zeros(B, c.intermediate_size, **f32)
        self.hid = torch.zeros(B, c.intermediate_size, **f32)
        self.logits = torch.zeros(B, c.vocab_size, **f32)
        self.meta = torch.zeros(3, B, device=dev, dtype=torch.int32)  # tokens, positions, slots
        self._slots: dict = {}
        self._free = list(range(self.n_slots - 1, -1, -1))

    # ---------------------------------------------------------------- requests
    def vocab_size(self) -> int:
        return self.cfg.vocab_size

    def evict(self, request_id: str) -> None:
        slot = self._slots.pop(request_id, None)
        if slot is not None:
            self._free.append(slot)

    def _slot(self, request_id: str) -> int:
        slot = self._slots.get(request_id)
        if slot is None:
            if not self._free:
                raise IllegalStateException(f"KV cache slots exhausted ({self.n_slots} live requests)")
            slot = self._free.pop()
            self.k_cache[:, slot].zero_()
            self.v_cache[:, slot].zero_()
            self._slots[request_id] = slot
        return slot

    # ---------------------------------------------------------------- forward
    def forward(self, request_id: str, tokens, start_pos: int) -> np.ndarray:
        return self.forward_batch([request_id], [tokens], [start_pos])[0]

    def forward_batch(self, request_ids, all_tokens, start_positions) -> list:
        n = len(request_ids)
        if len(all_tokens) != n or len(start_positions) != n:
            raise IllegalArgumentException(
                f"requestIds ({n}), allTokens ({len(all_tokens)}) and startPositions ({len(start_positions)}) "
                "must have the same size")
        if len(set(request_ids)) != n:
            raise IllegalArgumentException("a request may appear only once in a batch")
        toks, poss = [], []
        for rid, t, p in zip(request_ids, all_tokens, start_positions):
            t = np.asarray(t).reshape(-1)
            if t.size == 0:
                raise IllegalArgumentException(f"request {rid}: empty token array")
            if not 0 <= int(p) < self.max_seq:
                raise IllegalArgumentException(f"request {rid}: startPos {p} outside [0, {self.max_seq})")
            toks.append(int(np.clip(int(t[-1]), -2**31, 2**31 - 1)))
            poss.append(int(p))
        out = []
        for i in range(0, n, self.max_batch):
            out.extend(self._step(request_ids[i:i + self.max_batch], toks[i:i + self.max_batch],
                                  poss[i:i + self.max_batch]))
        return out

    def _step(self, rids, toks, poss) -> list:
        torch = _torch()
        B = len(rids)
        slots = [self._slot(r) for r in rids]
        self.meta[:, :B].copy_(torch.tensor([toks, poss, slots], dtype=torch.int32))
        self.enqueue(B)
        torch.cuda.synchronize()
        lg = self.logits[:B].cpu().numpy()
        return [lg[b].copy() for b in range(B)]

    def enqueue(self, B: int, stream=None) -> None:
        """One decode step for the first B requests of ``meta`` (tokens,
        positions, slots), on ``stream`` (a torch stream or None for the current)."""
        torch = _torch()
        c, L = self.cfg, self.L
        s = _V((stream or torch.cuda.current_stream()).cuda_stream)
        P = lambda t: _V(t.data_ptr())
        H, I, KV = c.hidden_dim, c.intermediate_size, c.kv_dim
        eps = c.rms_norm_eps

        def gemv(m, x, y):
            _check(L.jh_qmatvec_batched_dev(m.handle, P(x), B, P(y), 0, m.rows, s))

        def group(ms, x, ys):  # projections of one input: one launch on the MFMA path
            n = len(ms)
            hs = (_V * n)(*[m.handle for m in ms])
            xs = (_V * n)(*[P(x)] * n)
            yp = (_V * n)(*[P(y) for y in ys])
            _check(L.jh_qmatvec_batched_group_dev(n, hs, xs, B, yp, s))

        _check(L.jh_embed_rows_dev(self.w.token_embd.handle, P(self.meta[0]), B, P(self.x), s))
        for li, lw in enumerate(self.w.layers):
            res = None if li == 0 else P(self.proj)  # previous layer's ffn output (:784)
            _check(L.jh_rmsnorm_rows_dev(P(self.x), res, P(lw.attn_norm), H, B, eps, P(self.x), P(self.xn), s))
            m = lw.mats
            group([m["q"], m["k"], m["v"]], self.xn, [self.q, self.k, self.v])
            if lw.bias is not None:  # addInPlace of the projection biases (LlamaTransformerHandler.java:758-761)
                for name, out, n in (("q", self.q, H), ("k", self.k, KV), ("v", self.v, KV)):
                    _check(L.jh_add_rows_dev(P(out), P(lw.bias[name]), n, B, s))
            if self.lora is not None:  # applyLoraInPlace (LoraTrainableHandler.java:475-476)
                for proj, out in (("wq", self.q), ("wv", self.v)):
                    ad = self.lora.get(li, proj)
                    if ad is not None:
                        ad.apply_dev(self.xn.data_ptr(), out.data_ptr(), B, stream)
            _check(L.jh_rope_attention_batched_dev(P(self.q), P(self.k), P(self.v), B, c.num_heads, c.num_kv_heads,
                                                   c.head_dim, P(self.meta[1]), P(self.meta[2]), self.n_slots,
                                                   self.max_seq, c.rope_theta, P(self.k_cache[li]),
                                                   P(self.v_cache[li]), P(self.att), s))
            gemv(m["o"], self.att, self.proj)
            _check(L.jh_rmsnorm_rows_dev(P(self.x), P(self.proj), P(lw.ffn_norm), H, B, eps, P(self.x), P(self.xn),
                                         s))
            # silu(gate) * up (LlamaTransformerHandler.java:796-797): one launch pairs gate and up rows
            _check(L.jh_qmatvec_batched_swiglu_dev(m["gate"].handle, m["up"].handle, P(self.xn), B, P(self.hid),
                                                   P(self.gate), P(self.up), s))
            gemv(m["down"], self.hid, self.proj)
        _check(L.jh_rmsnorm_rows_dev(P(self.x), P(self.proj), P(self.w.output_norm), H, B, eps, P(self.x),
                                     P(self.xn), s))
        gemv(self.w.output, self.xn, self.logits)
