"""Device-resident Llama decode step over libjunohip.

Mirrors the reference's forward pass (paths under
/root/reference/node/src/main/java/cab/ml/juno/node/):

* ``LlamaConfig``      the LlamaConfig record (LlamaConfig.java:29-40; defaults
                       rmsNormEps 1e-5, ropeTheta 10000, :105-115)
* ``LlamaWeights``     the handler's per-layer tensors (attn / ffn norms and the
                       seven projections, LlamaTransformerHandler.java:743-800), the
                       output norm and output projection, device-resident and packed
* ``LlamaDecoder``     ``forward`` = getInitialActivation + runLayers +
                       outputProjection (LlamaTransformerHandler.java:603-810) for one
                       token at ``pos``, with the KV cache in HBM; ``capture`` records a
                       whole step as one HIP graph that advances the position on the
                       device, so steps replay without host work.

Each layer is the reference's transformerLayer: rmsNorm -> Q, K, V -> rope and
KV append -> gqa -> O + residual -> rmsNorm -> gate, up -> silu(gate) * up ->
down + residual.  The residual adds are fused into the following rmsNorm.
Everything runs on HIP kernels of libjunohip; there is no host fallback.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np

from . import _lib
from .matvec import (Q4_K, Q6_K, DeviceQuantMatrix, GpuContext, IllegalArgumentException, IllegalStateException,
                     _check)

_V = ctypes.c_void_p


def _torch():
    import torch  # device memory and streams: plumbing around the HIP library
    return torch


def _java_idiv(a: int, b: int) -> int:
    """Java int division (truncates toward zero); int overflow of a * 11 is
    not reproduced (hidden sizes are far below 2^31 / 11)."""
    q = abs(a) // abs(b)
    return q if (a >= 0) == (b >= 0) else -q


@dataclass
class LlamaConfig:
    hidden_dim: int
    num_layers: int
    num_heads: int
    num_kv_heads: int
    head_dim: int
    intermediate_size: int
    vocab_size: int
    rms_norm_eps: float = 1e-5
    rope_theta: float = 10000.0
    architecture: str = "llama"

    @classmethod
    def from_gguf(cls, r) -> "LlamaConfig":
        """LlamaConfig.from(GgufReader) (LlamaConfig.java:58-100): the architecture
        prefix's keys first, then the llama.* keys, then the reference's defaults;
        the vocabulary is the larger of the declared size and the length of
        tokenizer.ggml.tokens (LlamaConfig.java:106-109)."""
        arch = r.meta_string("general.architecture")
        if arch is None:
            arch = "llama"
        p = arch + "."
        hidden = r.meta_int(p + "embedding_length", r.meta_int("llama.embedding_length", 2048))
        layers = r.meta_int(p + "block_count", r.meta_int("llama.block_count", 22))
        heads = r.meta_int(p + "attention.head_count", r.meta_int("llama.attention.head_count", 32))
        kv_heads = r.meta_int(p + "attention.head_count_kv", r.meta_int("llama.attention.head_count_kv", heads))
        arch_vocab = r.meta_int(p + "vocab_size", r.meta_int("llama.vocab_size", 32000))
        toks = r.meta("tokenizer.ggml.tokens")
        tok_vocab = len(toks) if hasattr(toks, "elem_type") else 0
        vocab = max(arch_vocab, tok_vocab)
        ffn = r.meta_int(p + "feed_forward_length", r.meta_int("llama.feed_forward_length", _java_idiv(hidden * 11, 4)))
        eps = r.meta_float(p + "attention.layer_norm_rms_epsilon",
                           r.meta_float("llama.attention.layer_norm_rms_epsilon", 1e-5))
        theta = r.meta_float(p + "rope.freq_base", r.meta_float("llama.rope.freq_base", 10000.0))
        return cls(hidden, layers, heads, kv_heads, _java_idiv(hidden, heads), ffn, vocab, eps, theta, arch)

    @property
    def kv_dim(self) -> int:
        return self.num_kv_heads * self.head_dim

    @property
    def gqa_ratio(self) -> int:
        return self.num_heads // self.num_kv_heads

    def validate(self) -> None:
        if self.num_heads % self.num_kv_heads:
            raise IllegalArgumentException("numHeads must be a multiple of numKvHeads")
        if self.num_heads * self.head_dim != self.hidden_dim:
            raise IllegalArgumentException("numHeads * headDim must equal hiddenDim")


# Q4_K_M assignment used by the benchmark configs: Q6_K for attn_v, ffn_down
# and the output projection, Q4_K elsewhere.
Q4_K_M = {"q": Q4_K, "k": Q4_K, "v": Q6_K, "o": Q4_K, "gate": Q4_K, "up": Q4_K, "down": Q6_K, "output": Q6_K}


def matrix_shapes(cfg: LlamaConfig) -> dict:
    H, I, KV = cfg.hidden_dim, cfg.intermediate_size, cfg.kv_dim
    return {"q": (H, H), "k": (KV, H), "v": (KV, H), "o": (H, H), "gate": (I, H), "up": (I, H), "down": (H, I)}


@dataclass
class LlamaLayerWeights:
    attn_norm: object  # torch float32 [hidden] on the device
    ffn_norm: object
    mats: dict          # name -> DeviceQuantMatrix
    bias: dict | None = None  # "q" / "k" / "v" -> torch float32 projection bias (Qwen2), or None


@dataclass
class LlamaWeights:
    cfg: LlamaConfig
    layers: list
    output_norm: object
    output: DeviceQuantMatrix
    keep: list = field(default_factory=list)
    token_embd: DeviceQuantMatrix | None = None  # packed [vocab][hidden], for token input

    def close(self) -> None:
        for lw in self.layers:
            for m in lw.mats.values():
                m.close()
        self.output.close()
        if self.token_embd is not None and self.token_embd is not self.output:
            self.token_embd.close()

    # GGUF tensor names of a layer's projections (LlamaTransformerHandler.java:267-275)
    GGUF_NAMES = {"q": "attn_q", "k": "attn_k", "v": "attn_v", "o": "attn_output", "gate": "ffn_gate",
                  "up": "ffn_up", "down": "ffn_down"}

    @classmethod
    def from_gguf(cls, r, cfg: LlamaConfig | None = None, device: int = 0) -> "LlamaWeights":
        """Every layer of a GGUF model, streamed from the file into HBM packed
        (LlamaTransformerHandler.java:238-280, 459-470): blk.N.attn_norm /
        ffn_norm (F32 / F16 / BF16, widened on the host), the seven projections,
        the Q / K / V biases when the file has them (Qwen2, :258-280),
        output_norm, output.weight (token_embd.weight when the embeddings are
        tied) and token_embd.weight for token input."""
        torch = _torch()
        cfg = cfg or LlamaConfig.from_gguf(r)
        cfg.validate()
        has_bias = cfg.num_layers > 0 and r.has_tensor("blk.0.attn_q.bias")  # (LlamaTransformerHandler.java:258)
        be = GpuContext.shared(device).create_mat_vec()
        dev = torch.device("cuda", device)
        vec = lambda name: torch.from_numpy(np.ascontiguousarray(r.tensor(name), dtype=np.float32)).to(dev)
        shapes = matrix_shapes(cfg)
        made = []

        def mat(name, rows, cols):
            m = r.upload(name, be)
            made.append(m)
            if (m.rows, m.cols) != (rows, cols):
                raise IllegalArgumentException(
                    f"{name}: [{m.rows} x {m.cols}] on file, [{rows} x {cols}] expected from the config")
            return m

        try:
            layers = []
            for i in range(cfg.num_layers):
                mats = {m: mat(f"blk.{i}.{cls.GGUF_NAMES[m]}.weight", *shapes[m]) for m in shapes}
                bias = {m: vec(f"blk.{i}.attn_{m}.bias") for m in ("q", "k", "v")} if has_bias else None
                layers.append(LlamaLayerWeights(vec(f"blk.{i}.attn_norm.weight"), vec(f"blk.{i}.ffn_norm.weight"),
                                                mats, bias))
            embd = mat("token_embd.weight", cfg.vocab_size, cfg.hidden_dim) if r.has_tensor("token_embd.weight") \
                else None
            if r.has_tensor("output.weight"):
                out = mat("output.weight", cfg.vocab_size, cfg.hidden_dim)
            elif embd is not None:
                out = embd  # tied embeddings
            else:
                raise IllegalArgumentException("Tensor not found: output.weight (and no token_embd.weight)")
            return cls(cfg, layers, vec("output_norm.weight"), out, token_embd=embd)
        except BaseException:
            for m in made:
                m.close()
            raise

    @classmethod
    def random(cls, cfg: LlamaConfig, types: dict = Q4_K_M, seed: int = 0, device: int = 0,
               std: float = 0.02, embeddings: bool = False) -> "LlamaWeights":
        """Random-init weights ~ N(0, std) drawn on the device and packed with the
        device quantizer (bit-identical to LoraMerge's quantizers); norm weights
        1 + N(0, 0.1^2).  With embeddings, a Q6_K token_embd [vocab][hidden] ~ N(0, 1)
        for token input."""
        torch = _torch()
        cfg.validate()
        be = GpuContext.shared(device).create_mat_vec()
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        dev = torch.device("cuda", device)
        layers = []

        def qmat(qtype, rows, cols):
            w = torch.randn(rows * cols, generator=g, device=dev, dtype=torch.float32).mul_(std)
            m = be.quantize_dev(qtype, w.data_ptr(), rows, cols)
            torch.cuda.synchronize()
            del w
            return m

        def norm():
            return (1.0 + 0.1 * torch.randn(cfg.hidden_dim, generator=g, device=dev, dtype=torch.float32)).contiguous()

        shapes = matrix_shapes(cfg)
        for _ in range(cfg.num_layers):
            mats = {n: qmat(types[n], *shapes[n]) for n in shapes}
            layers.append(LlamaLayerWeights(norm(), norm(), mats))
        out = qmat(types["output"], cfg.vocab_size, cfg.hidden_dim)
        out_norm = norm()
        embd = None
        if embeddings:
            w = torch.randn(cfg.vocab_size * cfg.hidden_dim, generator=g, device=dev, dtype=torch.float32)
            embd = be.quantize_dev(Q6_K, w.data_ptr(), cfg.vocab_size, cfg.hidden_dim)
            torch.cuda.synchronize()
            del w
        return cls(cfg, layers, out_norm, out, token_embd=embd)

    @classmethod
    def from_packed(cls, cfg: LlamaConfig, layers: list, output_norm, output_raw, output_type: int,
                    device: int = 0) -> "LlamaWeights":
        """Upload packed GGUF tensors unchanged.  layers[i] holds 'attn_norm',
        'ffn_norm' (float32 [hidden]) and, per projection m in q k v o gate up down,
        'w' + m (packed bytes) and 'type_' + m."""
        torch = _torch()
        cfg.validate()
        be = GpuContext.shared(device).create_mat_vec()
        dev = torch.device("cuda", device)
        vec = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)
        shapes = matrix_shapes(cfg)
        out_layers = []
        for lw in layers:
            mats = {m: be.upload_quant(lw["type_" + m], *shapes[m], lw["w" + m]) for m in shapes}
            out_layers.append(LlamaLayerWeights(vec(lw["attn_norm"]), vec(lw["ffn_norm"]), mats))
        out = be.upload_quant(output_type, cfg.vocab_size, cfg.hidden_dim, output_raw)
        return cls(cfg, out_layers, vec(output_norm), out)


class LlamaDecoder:
    """One request's decode state: KV cache [layers][max_seq][kv_dim] in HBM,
    activation buffers and the device position."""

    def __init__(self, weights: LlamaWeights, max_seq: int, device: int = 0, lora=None):
        torch = _torch()
        self.w, self.cfg, self.max_seq = weights, weights.cfg, max_seq
        self.lora = lora  # LoraAdapterSet: "wq" / "wv" deltas after the Q and V projections
        c = self.cfg
        self.L = _lib.load()
        dev = torch.device("cuda", device)
        f32 = dict(device=dev, dtype=torch.float32)
        self.k_cache = torch.zeros(c.num_layers, max_seq, c.kv_dim, **f32)
        self.v_cache = torch.zeros(c.num_layers, max_seq, c.kv_dim, **f32)
        self.x = torch.zeros(c.hidden_dim, **f32)      # residual stream (the step's input activation)
        self.x2 = torch.zeros(c.hidden_dim, **f32)     # its ping-pong twin: a fused norm writes h = x + res here
        self.xn = torch.zeros(c.hidden_dim, **f32)     # normalised input of a projection
        self.q = torch.zeros(c.hidden_dim, **f32)
        self.k = torch.zeros(c.kv_dim, **f32)
        self.v = torch.zeros(c.kv_dim, **f32)
        self.att = torch.zeros(c.hidden_dim, **f32)
        self.proj = torch.zeros(c.hidden_dim, **f32)
        self.hid = torch.zeros(c.intermediate_size, **f32)
        self.logits = torch.zeros(c.vocab_size, **f32)
        self.pos = torch.zeros(1, device=dev, dtype=torch.int32)
        self.token = torch.zeros(1, device=dev, dtype=torch.int32)  # input token of a token step

    # ---------------------------------------------------------------- enqueue
    def _group(self, mats, xs, ys, s) -> None:
        n = len(mats)
        handles = (_V * n)(*[m.handle for m in mats])
        dx = (_V * n)(*[x.data_ptr() for x in xs])
        dy = (_V * n)(*[y.data_ptr() for y in ys])
        _check(self.L.jh_qmatvec_group_dev(n, handles, dx, dy, s))

    def enqueue_step(self, stream=None, advance: bool = False, from_token: bool = False) -> None:
        """Enqueue one decode step on ``stream`` (a torch stream or None for the
        current one): x (the input activation) -> logits at position *pos.  With
        from_token, x is first set to the embedding row of *token.  With
        advance, *pos += 1 on the device at the end (for graph replay)."""
        torch = _torch()
        c, L = self.cfg, self.L
        s = _V((stream or torch.cuda.current_stream()).cuda_stream)
        P = lambda t: _V(t.data_ptr())
        if from_token:  # getInitialActivation (LlamaTransformerHandler.java:651-660)
            if self.w.token_embd is None:
                raise IllegalStateException("no token_embd.weight: this node takes activations")
            _check(L.jh_embed_dev(self.w.token_embd.handle, P(self.token), P(self.x), s))
        eps, nh, nkv, hd, H = c.rms_norm_eps, c.num_heads, c.num_kv_heads, c.head_dim, c.hidden_dim
        # The residual stream alternates between x and x2: the norms are fused
        # into the q / k / v and gate / up launches, whose workgroups all read the
        # residual while one of them writes the sum, so the sum goes to the other
        # buffer.
        cur, other = self.x, self.x2
        for li, lw in enumerate(self.w.layers):
            m = lw.mats
            if li == 0:  # rmsNorm(x) (LlamaTransformerHandler.java:748)
                _check(L.jh_rmsnorm_dev(P(cur), None, P(lw.attn_norm), H, eps, None, P(self.xn), s))
                self._group([m["q"], m["k"], m["v"]], [self.xn] * 3, [self.q, self.k, self.v], s)
            elif self.lora is not None:  # the adapters read the normalised input: keep it in xn
                _check(L.jh_rmsnorm_dev(P(cur), P(self.proj), P(lw.attn_norm), H, eps, P(cur), P(self.xn), s))
                self._group([m["q"], m["k"], m["v"]], [self.xn] * 3, [self.q, self.k, self.v], s)
            else:
                # previous layer's x2 + ffnOut (:784), this layer's rmsNorm and the q / k / v
                # projections (:748-757) in one launch where it applies; the sum goes to the
                # other residual buffer (the launch's workgroups all read this one)
                qkv = [m["q"], m["k"], m["v"]]
                _check(L.jh_rmsnorm_qmatvec_group_dev(3, (_V * 3)(*[q.handle for q in qkv]), P(cur), P(self.proj),
                                                      P(lw.attn_norm), eps, P(other), P(self.xn),
                                                      (_V * 3)(P(self.q), P(self.k), P(self.v)), s))
                cur, other = other, cur
            if lw.bias is not None:  # addInPlace of the projection biases (:758-761)
                for name, out in (("q", self.q), ("k", self.k), ("v", self.v)):
                    _check(L.jh_add_rows_dev(P(out), P(lw.bias[name]), out.numel(), 1, s))
            if self.lora is not None:  # applyLoraInPlace (LoraTrainableHandler.java:475-476)
                for proj, out in (("wq", self.q), ("wv", self.v)):
                    ad = self.lora.get(li, proj)
                    if ad is not None:
                        ad.apply_dev(self.xn.data_ptr(), out.data_ptr(), 1, stream)
            # rope on q and k, KV append, gqa (:765-773) and the output projection (:776): the
            # attention combine runs in the projection's input conversion where that applies
            _check(L.jh_rope_attention_qmatvec_dev(P(self.q), P(self.k), P(self.v), nh, nkv, hd, P(self.pos),
                                                   self.max_seq, c.rope_theta, P(self.k_cache[li]),
                                                   P(self.v_cache[li]), m["o"].handle, P(self.att), P(self.proj), s))
            # x2 = x + attnProj (:778), rmsNorm(x2) (:781) and silu(gate . x2n) * (up . x2n) (:796-797):
            # where the staged kernel applies, one launch (the norm in its input conversion, each gate row
            # paired with its up row); else the norm into xn and the paired GEMV
            _check(L.jh_rmsnorm_qmatvec_swiglu_dev(m["gate"].handle, m["up"].handle, P(cur), P(self.proj),
                                                   P(lw.ffn_norm), eps, P(other), P(self.xn), P(self.hid), s))
            cur, other = other, cur
            self._group([m["down"]], [self.hid], [self.proj], s)
        # final residual, rmsNorm(x, outputNorm) and the output projection (:803-810), fused the same way
        _check(L.jh_rmsnorm_qmatvec_dev(self.w.output.handle, P(cur), P(self.proj), P(self.w.output_norm), eps,
                                        P(other), P(self.xn), P(self.logits), s))
        if advance:
            _check(L.jh_pos_increment_dev(P(self.pos), 1, s))

    # ---------------------------------------------------------------- host API
    def forward(self, activation, pos: int) -> np.ndarray:
        """logits for one token whose input activation (the embedding row, or the
        previous node's activations) is ``activation`` at position ``pos``."""
        torch = _torch()
        a = np.ascontiguousarray(activation, dtype=np.float32).reshape(-1)
        if a.size != self.cfg.hidden_dim:
            raise IllegalArgumentException(f"activation length {a.size} != hiddenDim {self.cfg.hidden_dim}")
        if not 0 <= pos < self.max_seq:
            raise IllegalArgumentException(f"pos {pos} outside [0, {self.max_seq})")
        self.x.copy_(torch.from_numpy(a))
        self.pos.fill_(pos)
        self.enqueue_step()
        torch.cuda.synchronize()
        return self.logits.cpu().numpy()

    def forward_token(self, token: int, pos: int) -> np.ndarray:
        """logits for ``token`` at ``pos`` (the embedding row, clamped to the
        vocabulary as getInitialActivation does, is the input activation)."""
        torch = _torch()
        if not 0 <= pos < self.max_seq:
            raise IllegalArgumentException(f"pos {pos} outside [0, {self.max_seq})")
        self.token.fill_(int(np.clip(token, -2**31, 2**31 - 1)))
        self.pos.fill_(pos)
        self.enqueue_step(from_token=True)
        torch.cuda.synchronize()
        return self.logits.cpu().numpy()

    def capture(self, stream, from_token: bool = False):
        """A HIP graph of one step that also advances *pos; replay it after
        writing the next activation into ``self.x`` (or, with from_token, the next
        token into ``self.token``).  Capturing runs one eager
        warm-up step first (it allocates the library's stream workspace outside
        the capture), which overwrites x, the logits and the KV row at *pos."""
        torch = _torch()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            self.enqueue_step(stream, from_token=from_token)  # warm-up: workspaces are allocated outside the capture
            stream.synchronize()
            with torch.cuda.graph(g, stream=stream):
                self.enqueue_step(stream, advance=True, from_token=from_token)
        return g
