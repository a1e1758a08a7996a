"""forwardBatch on the device (juno_amd/pipeline.py): N requests stacked
through every layer in one pass (batched GEMVs, batched rope + KV append +
attention over per-request cache slots) against N single-request decoders
(InferencePipeline.forwardBatch's default, a serial loop over forward(),
InferencePipeline.java:62-69) and against the oracle's transformerLayer.

Tolerance: logits within 1e-3 of max|logit| (the batched kernels differ from
the B = 1 kernels in the order of fp32 sums, and the MFMA path at B >= 3 in
x's hi/lo fp16 split, both inside the GEMV bar).
"""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from juno_amd import decode as D  # noqa: E402
from juno_amd.matvec import IllegalArgumentException, IllegalStateException  # noqa: E402
from juno_amd.pipeline import LlamaBatchPipeline  # noqa: E402

CFG = D.LlamaConfig(hidden_dim=256, num_layers=2, num_heads=4, num_kv_heads=2, head_dim=64, intermediate_size=512,
                    vocab_size=1000)


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def weights():
    w = D.LlamaWeights.random(CFG, seed=31, embeddings=True)
    yield w
    w.close()


def err(a, b):
    return float(np.abs(a.astype(np.float64) - b).max() / np.abs(b).max())


def test_forward_batch_matches_serial_forward(weights):
    """Requests join and leave over the steps, so the batch mixes positions;
    B runs through the GEMV-kernel sizes and the MFMA sizes (>= 16)."""
    pipe = LlamaBatchPipeline(weights, max_seq=32, max_batch=24)
    serial = {}
    rng = np.random.default_rng(5)
    pos = {}
    schedule = [list(range(3)), list(range(5)), list(range(20)), [0, 4, 7, 19, 21], list(range(22))]
    for step, members in enumerate(schedule):
        rids = [f"r{i}" for i in members]
        toks = [[int(rng.integers(0, CFG.vocab_size))] for _ in rids]
        poss = [pos.get(r, 0) for r in rids]
        say("batch step", step, "B =", len(rids))
        got = pipe.forward_batch(rids, toks, poss)
        assert len(got) == len(rids) and all(g.shape == (CFG.vocab_size,) for g in got)
        for r, t, p, g in zip(rids, toks, poss, got):
            if r not in serial:
                serial[r] = D.LlamaDecoder(weights, max_seq=32)
            ref = serial[r].forward_token(t[-1], p)
            assert err(g, ref) <= 1e-3, (step, r, err(g, ref))
            pos[r] = p + 1


def test_forward_batch_vs_oracle(weights):
    pipe = LlamaBatchPipeline(weights, max_seq=16, max_batch=4)
    layers = []
    for lw in weights.layers:
        d = {"attn_norm": lw.attn_norm.cpu().numpy(), "ffn_norm": lw.ffn_norm.cpu().numpy()}
        for m, mat in lw.mats.items():
            d["w" + m], d["type_" + m] = mat.packed_bytes(), mat.type
        layers.append(d)
    out_norm, out_raw = weights.output_norm.cpu().numpy(), weights.output.packed_bytes()
    table = O.dequantize(O.Q6_K, weights.token_embd.packed_bytes(), CFG.vocab_size, CFG.hidden_dim)
    dims = dict(hidden=CFG.hidden_dim, n_heads=CFG.num_heads, n_kv_heads=CFG.num_kv_heads, head_dim=CFG.head_dim,
                ffn=CFG.intermediate_size, eps=CFG.rms_norm_eps, theta=CFG.rope_theta)
    caches = {r: (np.zeros((CFG.num_layers, 16, CFG.kv_dim), np.float32),
                  np.zeros((CFG.num_layers, 16, CFG.kv_dim), np.float32)) for r in ("a", "b", "c")}
    tok_seq = {"a": [5, 9, 13], "b": [700, 1, 999], "c": [42, 42, 42]}
    for p in range(3):
        got = pipe.forward_batch(["a", "b", "c"], [[tok_seq[r][p]] for r in "abc"], [p, p, p])
        for r, g in zip("abc", got):
            x = table[tok_seq[r][p]]
            kc, vc = caches[r]
            for li, lw in enumerate(layers):
                x = O.llama_layer(lw, dims, x, p, kc[li], vc[li])
            ref = O.matvec(O.Q6_K, out_raw, O.rmsnorm(x, out_norm, CFG.rms_norm_eps), 0, CFG.vocab_size,
                           CFG.hidden_dim)
            assert err(g, ref) <= 1e-3, (p, r, err(g, ref))


def test_forward_is_forward_batch_of_one_and_chunking(weights):
    pipe = LlamaBatchPipeline(weights, max_seq=8, max_batch=3, max_requests=8)
    one = pipe.forward("solo", [1, 2, 3], 0)  # the last token is the input
    pipe.evict("solo")
    again = pipe.forward_batch(["solo"], [[3]], [0])[0]
    assert np.array_equal(one, again)
    # 7 requests with max_batch 3: three device steps, results in request order
    rids = [f"q{i}" for i in range(7)]
    got = pipe.forward_batch(rids, [[i * 11] for i in range(7)], [0] * 7)
    ref = LlamaBatchPipeline(weights, max_seq=8, max_batch=8).forward_batch(rids, [[i * 11] for i in range(7)],
                                                                             [0] * 7)
    for g, r in zip(got, ref):
        assert err(g, r) <= 1e-3


def test_evicted_slot_is_clean_for_the_next_request(weights):
    pipe = LlamaBatchPipeline(weights, max_seq=8, max_batch=2, max_requests=2)
    for p in range(4):
        pipe.forward_batch(["old1", "old2"], [[p + 1], [p + 2]], [p, p])
    pipe.evict("old1")
    # a new request that starts at position 2 reads zeros at 0..1, as a fresh cache would
    got = pipe.forward("new", [77], 2)
    fresh = LlamaBatchPipeline(weights, max_seq=8, max_batch=1, max_requests=1).forward("x", [77], 2)
    assert np.array_equal(got, fresh)
    with pytest.raises(IllegalStateException, match="slots exhausted"):
        pipe.forward("third", [1], 0)


def test_forward_batch_arguments(weights):
    pipe = LlamaBatchPipeline(weights, max_seq=8, max_batch=2)
    assert pipe.vocab_size() == CFG.vocab_size
    assert pipe.forward_batch([], [], []) == []
    with pytest.raises(IllegalArgumentException, match="same size"):
        pipe.forward_batch(["a", "b"], [[1]], [0, 0])
    with pytest.raises(IllegalArgumentException, match="only once"):
        pipe.forward_batch(["a", "a"], [[1], [2]], [0, 1])
    with pytest.raises(IllegalArgumentException, match="empty token"):
        pipe.forward("a", [], 0)
    with pytest.raises(IllegalArgumentException, match="startPos"):
        pipe.forward("a", [1], 8)
