"""GGUF files into HBM on the GPU: jh_gguf_upload streams a tensor from the
file into a resident matrix (bytes identical to tensorRaw + upload), packed
tensors dequantize bit-exactly through GgufReader.tensor (the reference's
known-answer blocks, GgufReaderTest.java:60-105, 334-358, 634-653), the
embedding lookup matches getInitialActivation (LlamaTransformerHandler.java:
651-660, token clamped), and a whole model loaded from a GGUF file decodes
like the same weights uploaded from memory and like the oracle.
"""
import ctypes
import struct

import numpy as np
import pytest

import oracle as O
from gguf_build import ARRAY, FLOAT32, STRING, UINT32, gguf_bytes, llamafile, minimal_gguf

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from juno_amd import GgufReader, GpuContext, UnsupportedOperationException  # noqa: E402
from juno_amd import decode as D  # noqa: E402
from juno_amd import _lib  # noqa: E402


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def be():
    return GpuContext.shared(0).create_mat_vec()


def rand_packed(qtype, rows, cols, seed):
    w = (np.random.default_rng(seed).standard_normal(rows * cols) * 0.02).astype(np.float32)
    return O.quantize(qtype, w)


@pytest.mark.parametrize("qtype,rows,cols", [(O.Q4_K, 96, 512), (O.Q5_K, 40, 768), (O.Q6_K, 33, 256),
                                             (O.Q8_0, 17, 96), (O.F32, 5, 64)])
def test_upload_streams_the_tensor_bytes(be, tmp_path, qtype, rows, cols):
    say("gguf upload", qtype, rows, cols)
    raw = rand_packed(qtype, rows, cols, rows) if qtype != O.F32 else \
        np.random.default_rng(1).standard_normal(rows * cols).astype(np.float32).view(np.uint8)
    p = tmp_path / "m.llamafile"
    p.write_bytes(llamafile("m.gguf", gguf_bytes((), [("pad", [3], 0, bytes(12)), ("w", [cols, rows], qtype,
                                                                                   raw.tobytes())])))
    with GgufReader.open(p) as r:
        m = r.upload("w", be)
        assert (m.type, m.rows, m.cols) == (qtype, rows, cols)
        assert np.array_equal(m.packed_bytes(), raw)
        x = np.random.default_rng(2).standard_normal(cols).astype(np.float32)
        ref_m = be.upload_quant(qtype, rows, cols, raw)
        assert np.array_equal(be.sgemv_quant(m, x), be.sgemv_quant(ref_m, x))  # same bytes, same kernel
        if qtype != O.F32:
            assert np.array_equal(r.tensor("w", be).reshape(rows, cols).view(np.uint32),
                                  O.dequantize(qtype, raw, rows, cols).view(np.uint32))
        m.close()
        ref_m.close()


def test_large_tensor_streams_in_chunks(be, tmp_path):
    cols = 14336  # about 2.5 of the loader's 32 MiB staging chunks, and a ragged last one
    rows = 5 * (32 << 20) // 2 // (cols // 256 * 144) + 7
    say("gguf large upload", rows, cols)
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    w = torch.randn(rows * cols, generator=g, device="cuda").mul_(0.02)
    src = be.quantize_dev(O.Q4_K, w.data_ptr(), rows, cols)
    torch.cuda.synchronize()
    del w
    raw = src.packed_bytes()
    p = tmp_path / "big.gguf"
    p.write_bytes(gguf_bytes((), [("w", [cols, rows], O.Q4_K, raw.tobytes())]))
    with GgufReader.open(p) as r:
        m = r.upload("w", be)
        assert np.array_equal(m.packed_bytes(), raw)
        m.close()
    src.close()


def test_reference_known_answer_blocks_through_a_file(be, tmp_path, golden):
    g = golden["q6k_golden_block"]
    blk = np.zeros(210, dtype=np.uint8)
    blk[:128] = np.array(g["ql"]).astype(np.int8).view(np.uint8)
    blk[128:192] = np.array(g["qh"]).astype(np.int8).view(np.uint8)
    blk[192:208] = np.array(g["sc"]).astype(np.int8).view(np.uint8)
    blk[208:] = [g["d_f16"] & 0xFF, g["d_f16"] >> 8]
    z = golden["q4k_all_zero"]
    q4 = struct.pack("<HH", z["d_f16"], z["dmin_f16"]) + bytes(140)
    q8 = struct.pack("<H", golden["q8_0_llamafile"]["scale_f16"]) + bytes(range(32))
    p = tmp_path / "ka.llamafile"
    p.write_bytes(llamafile("ka.gguf", gguf_bytes((), [("q6", [256], 14, blk.tobytes()), ("q4", [256], 12, q4),
                                                         ("q8", [32], 8, q8)])))
    with GgufReader.open(p) as r:
        out = r.tensor("q6", be)
        for idx, val in g["expected"].items():
            assert out[int(idx)] == np.float32(val)
        assert np.all(r.tensor("q4", be) == 0.0)
        assert np.array_equal(r.tensor("q8", be), (0.5 * np.arange(32)).astype(np.float32))


def test_upload_errors(be, tmp_path):
    p = tmp_path / "e.gguf"
    p.write_bytes(gguf_bytes((), [("q40", [256], 2, bytes(144)), ("odd", [100, 2], 12, bytes(0))]))
    with GgufReader.open(p) as r:
        with pytest.raises(UnsupportedOperationException):
            r.upload("q40", be)  # Q4_0: sized by rawByteCount, but the reference has no matVec for it
        with pytest.raises(Exception, match="multiple of the block size"):
            r.upload("odd", be)


# ------------------------------------------------------------------ embedding lookup

@pytest.mark.parametrize("qtype", [O.Q4_K, O.Q6_K, O.Q8_0, O.Q5_K])
def test_embed_row_clamps_like_getInitialActivation(be, qtype):
    L = _lib.load()
    vocab, hidden = 77, 512
    raw = rand_packed(qtype, vocab, hidden, 9)
    m = be.upload_quant(qtype, vocab, hidden, raw)
    table = O.dequantize(qtype, raw, vocab, hidden)
    out = torch.full((hidden,), float("nan"), device="cuda")
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    for t, want in [(0, 0), (5, 5), (76, 76), (77, 76), (10**6, 76), (-1, 0), (-(2**31), 0)]:
        say("embed", qtype, t)
        tok.fill_(t)
        assert L.jh_embed_dev(m.handle, ctypes.c_void_p(tok.data_ptr()), ctypes.c_void_p(out.data_ptr()), None) == 0
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy().view(np.uint32), table[want].view(np.uint32)), t
    m.close()


# ------------------------------------------------------------------ a model from a GGUF file

CFG = D.LlamaConfig(hidden_dim=256, num_layers=2, num_heads=4, num_kv_heads=2, head_dim=64, intermediate_size=512,
                    vocab_size=1000)


def model_gguf(cfg, seed, tied=False, extra_tokens=0, bias=False):
    """A GGUF model (Q4_K_M assignment) with llama.* metadata, optionally with
    Q / K / V biases (Qwen2); returns the file bytes and the host tensors for
    the oracle."""
    rng = np.random.default_rng(seed)
    shapes = D.matrix_shapes(cfg)
    tensors, layers = [], []
    f32 = lambda a: np.ascontiguousarray(a, np.float32)
    for i in range(cfg.num_layers):
        lw = {"attn_norm": f32(1 + 0.1 * rng.standard_normal(cfg.hidden_dim)),
              "ffn_norm": f32(1 + 0.1 * rng.standard_normal(cfg.hidden_dim))}
        tensors.append((f"blk.{i}.attn_norm.weight", [cfg.hidden_dim], 0, lw["attn_norm"].tobytes()))
        for m, (rows, cols) in shapes.items():
            t = D.Q4_K_M[m]
            lw["w" + m], lw["type_" + m] = O.quantize(t, f32(rng.standard_normal(rows * cols) * 0.02)), t
            tensors.append((f"blk.{i}.{D.LlamaWeights.GGUF_NAMES[m]}.weight", [cols, rows], t, lw["w" + m].tobytes()))
        tensors.append((f"blk.{i}.ffn_norm.weight", [cfg.hidden_dim], 0, lw["ffn_norm"].tobytes()))
        if bias:
            for m, n in (("q", cfg.hidden_dim), ("k", cfg.kv_dim), ("v", cfg.kv_dim)):
                lw["b" + m] = f32(rng.standard_normal(n) * 0.5)
                tensors.append((f"blk.{i}.attn_{m}.bias", [n], 0, lw["b" + m].tobytes()))
        layers.append(lw)
    out_norm = f32(1 + 0.1 * rng.standard_normal(cfg.hidden_dim))
    embd = O.quantize(O.Q6_K, f32(rng.standard_normal(cfg.vocab_size * cfg.hidden_dim)))
    tensors += [("token_embd.weight", [cfg.hidden_dim, cfg.vocab_size], O.Q6_K, embd.tobytes()),
                ("output_norm.weight", [cfg.hidden_dim], 0, out_norm.tobytes())]
    out_raw = embd
    if not tied:
        out_raw = O.quantize(O.Q6_K, f32(rng.standard_normal(cfg.vocab_size * cfg.hidden_dim) * 0.02))
        tensors.append(("output.weight", [cfg.hidden_dim, cfg.vocab_size], O.Q6_K, out_raw.tobytes()))
    meta = [("general.architecture", STRING, "llama"), ("llama.embedding_length", UINT32, cfg.hidden_dim),
            ("llama.block_count", UINT32, cfg.num_layers), ("llama.attention.head_count", UINT32, cfg.num_heads),
            ("llama.attention.head_count_kv", UINT32, cfg.num_kv_heads),
            ("llama.feed_forward_length", UINT32, cfg.intermediate_size),
            ("llama.vocab_size", UINT32, cfg.vocab_size - extra_tokens),
            ("llama.attention.layer_norm_rms_epsilon", FLOAT32, cfg.rms_norm_eps),
            ("llama.rope.freq_base", FLOAT32, cfg.rope_theta),
            ("tokenizer.ggml.tokens", ARRAY, (STRING, [f"<{i}>" for i in range(cfg.vocab_size)]))]
    return gguf_bytes(meta, tensors), layers, out_norm, out_raw, embd


def oracle_logits(cfg, layers, out_norm, out_raw, x, pos, kc, vc):
    dims = dict(hidden=cfg.hidden_dim, n_heads=cfg.num_heads, n_kv_heads=cfg.num_kv_heads, head_dim=cfg.head_dim,
                ffn=cfg.intermediate_size, eps=cfg.rms_norm_eps, theta=cfg.rope_theta)
    for li, lw in enumerate(layers):
        x = O.llama_layer(lw, dims, x, pos, kc[li], vc[li])
    return O.matvec(O.Q6_K, out_raw, O.rmsnorm(x, out_norm, cfg.rms_norm_eps), 0, cfg.vocab_size, cfg.hidden_dim)


@pytest.mark.parametrize("tied", [False, True])
def test_model_from_gguf_decodes_tokens(tmp_path, tied):
    data, layers, out_norm, out_raw, embd = model_gguf(CFG, 21, tied=tied, extra_tokens=24)
    p = tmp_path / "tiny.gguf"
    p.write_bytes(data)
    with GgufReader.open(p) as r:
        cfg = D.LlamaConfig.from_gguf(r)
        assert cfg.vocab_size == CFG.vocab_size  # the tokenizer's count wins over llama.vocab_size
        say("gguf model load, tied =", tied)
        w = D.LlamaWeights.from_gguf(r, cfg)
    assert (w.output is w.token_embd) == tied
    w_mem = D.LlamaWeights.from_packed(cfg, layers, out_norm, out_raw, O.Q6_K)
    dec, dec_mem = D.LlamaDecoder(w, max_seq=32), D.LlamaDecoder(w_mem, max_seq=32)
    table = O.dequantize(O.Q6_K, embd, cfg.vocab_size, cfg.hidden_dim)
    kc = np.zeros((cfg.num_layers, 32, cfg.kv_dim), np.float32)
    vc = np.zeros_like(kc)
    for pos, tok in enumerate([1, 999, 5000, -3, 42]):
        say("gguf token step", pos, tok)
        got = dec.forward_token(tok, pos)
        x = table[min(max(tok, 0), cfg.vocab_size - 1)]
        assert np.array_equal(got, dec_mem.forward(x, pos))  # same bytes, same kernels: bit-identical
        ref = oracle_logits(cfg, layers, out_norm, out_raw, x, pos, kc, vc)
        err = np.abs(got.astype(np.float64) - ref).max() / np.abs(ref).max()
        assert err <= 1e-3, (pos, err)
    w.close()
    w_mem.close()


def test_token_graph_replay_matches_eager(tmp_path):
    data = model_gguf(CFG, 22)[0]
    p = tmp_path / "tiny.gguf"
    p.write_bytes(data)
    with GgufReader.open(p) as r:
        w = D.LlamaWeights.from_gguf(r)
    eager, graph = D.LlamaDecoder(w, max_seq=16), D.LlamaDecoder(w, max_seq=16)
    s = torch.cuda.Stream()
    g = graph.capture(s, from_token=True)
    graph.pos.fill_(0)
    for pos, tok in enumerate([3, 7, 7, 900]):
        say("gguf token replay", pos)
        ref = eager.forward_token(tok, pos)
        with torch.cuda.stream(s):
            graph.token.fill_(tok)
            g.replay()
        s.synchronize()
        assert np.array_equal(graph.logits.cpu().numpy(), ref), pos
    w.close()


def oracle_logits_bias(cfg, layers, out_norm, out_raw, x, pos, kc, vc):
    """transformerLayer with the projection biases (LlamaTransformerHandler.java:743-800,
    addInPlace :758-761) composed from the oracle's pieces."""
    nh, nkv, hd, eps = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.rms_norm_eps
    mv = lambda lw, m, v: O.matvec(lw["type_" + m], lw["w" + m], v, 0, *D.matrix_shapes(cfg)[m])
    for li, lw in enumerate(layers):
        xn = O.rmsnorm(x, lw["attn_norm"], eps)
        q, k, v = (O.add(mv(lw, m, xn), lw["b" + m]) for m in ("q", "k", "v"))
        q, k = O.rope(q, pos, nh, hd, cfg.rope_theta), O.rope(k, pos, nkv, hd, cfg.rope_theta)
        kc[li][pos], vc[li][pos] = k, v
        x2 = O.add(x, mv(lw, "o", O.gqa(q, kc[li], vc[li], nh, nkv, hd, pos + 1)))
        xn2 = O.rmsnorm(x2, lw["ffn_norm"], eps)
        x = O.add(x2, mv(lw, "down", O.silu_mul(mv(lw, "gate", xn2), mv(lw, "up", xn2))))
    return O.matvec(O.Q6_K, out_raw, O.rmsnorm(x, out_norm, eps), 0, cfg.vocab_size, cfg.hidden_dim)


def test_qwen2_style_biases_from_gguf(tmp_path):
    """Q / K / V biases (Qwen2AttentionBiasTest.java, LlamaTransformerHandler.java:258-280, 758-761),
    single-request and batched."""
    data, layers, out_norm, out_raw, embd = model_gguf(CFG, 23, bias=True)
    p = tmp_path / "qwen2ish.gguf"
    p.write_bytes(data)
    with GgufReader.open(p) as r:
        w = D.LlamaWeights.from_gguf(r)
    assert all(lw.bias is not None for lw in w.layers)
    dec = D.LlamaDecoder(w, max_seq=8)
    table = O.dequantize(O.Q6_K, embd, CFG.vocab_size, CFG.hidden_dim)
    kc = np.zeros((CFG.num_layers, 8, CFG.kv_dim), np.float32)
    vc = np.zeros_like(kc)
    for pos, tok in enumerate([5, 600, 17]):
        got = dec.forward_token(tok, pos)
        ref = oracle_logits_bias(CFG, layers, out_norm, out_raw, table[tok], pos, kc, vc)
        err = np.abs(got.astype(np.float64) - ref).max() / np.abs(ref).max()
        assert err <= 1e-3, (pos, err)
    from juno_amd.pipeline import LlamaBatchPipeline
    pipe = LlamaBatchPipeline(w, max_seq=8, max_batch=4)
    solo = [D.LlamaDecoder(w, max_seq=8) for _ in range(2)]
    for pos in range(2):
        got = pipe.forward_batch(["x", "y"], [[9 + pos], [800]], [pos, pos])
        for dec_i, t, g in zip(solo, [9 + pos, 800], got):
            ref = dec_i.forward_token(t, pos)
            assert np.abs(g - ref).max() <= 1e-3 * np.abs(ref).max()
    w.close()
