"""GPU parity of the device-resident decode step (jh_decode.hip through the
C-ABI, juno_amd/decode.py) against the CPU oracle's restatement of
LlamaTransformerHandler (oracle/juno_oracle_decode.c).

Tolerances: rmsnorm / rope / silu are elementwise fp32 with double-precision
transcendentals like the reference: within 2e-6 relative (a few ulp).  gqa
and the whole step differ from the reference only in the order of fp32 sums
(and the GEMVs' 1e-3 bar): attention outputs within 1e-5 of max|out|; step
logits held to the GEMV bar per row (|err| / max(|ref|, 1e-3 sum_c |w_rc xn_c|)
<= 1e-3, with the oracle's normed final x) after several layers and positions.
"""
import ctypes

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from juno_amd import _lib  # noqa: E402
from juno_amd import decode as D  # noqa: E402
from juno_amd.matvec import IllegalArgumentException  # noqa: E402

V = ctypes.c_void_p


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def L():
    return _lib.load()


def dev(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda", dtype)


def vec(n, seed, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(n) * scale).astype(np.float32)


def P(t):
    return V(t.data_ptr())


# ------------------------------------------------------------------ ops

@pytest.mark.parametrize("n", [64, 2048, 4096, 5000])
def test_rmsnorm_with_residual(L, n):
    say("rmsnorm", n)
    x, r, w = vec(n, 1), vec(n, 2), vec(n, 3)
    dx, dr, dw = dev(x), dev(r), dev(w)
    out = torch.empty(n, device="cuda")
    assert L.jh_rmsnorm_dev(P(dx), None, P(dw), n, 1e-5, None, P(out), None) == 0
    ref = O.rmsnorm(x, w, 1e-5)
    assert np.allclose(out.cpu().numpy(), ref, rtol=2e-6, atol=1e-7)
    # fused residual, written in place (x_out == x)
    assert L.jh_rmsnorm_dev(P(dx), P(dr), P(dw), n, 1e-5, P(dx), P(out), None) == 0
    torch.cuda.synchronize()
    assert np.array_equal(dx.cpu().numpy(), O.add(x, r))
    assert np.allclose(out.cpu().numpy(), O.rmsnorm(O.add(x, r), w, 1e-5), rtol=2e-6, atol=1e-7)


def test_rmsnorm_arguments(L):
    d = torch.zeros(16, device="cuda")
    assert L.jh_rmsnorm_dev(P(d), None, P(d), 0, 1e-5, None, P(d), None) != 0
    assert L.jh_rmsnorm_dev(P(d), None, P(d), 16, 1e-5, None, P(d), None) != 0  # out aliases x
    assert b"alias" in L.jh_last_error()


@pytest.mark.parametrize("nh,nkv,hd", [(32, 4, 64), (32, 8, 128), (8, 8, 64)])
def test_rope_kv_append(L, nh, nkv, hd):
    say("rope_kv", nh, nkv, hd)
    max_seq, theta = 600, 10000.0
    kvd = nkv * hd
    kc = torch.zeros(max_seq, kvd, device="cuda")
    vc = torch.zeros(max_seq, kvd, device="cuda")
    for pos in (0, 1, 37, 511, 599):
        q, k, v = vec(nh * hd, pos), vec(kvd, pos + 1), vec(kvd, pos + 2)
        dq, dk, dv = dev(q), dev(k), dev(v)
        dpos = torch.tensor([pos], dtype=torch.int32, device="cuda")
        assert L.jh_rope_kv_dev(P(dq), P(dk), P(dv), nh, nkv, hd, P(dpos), max_seq, theta, P(kc), P(vc), None) == 0
        torch.cuda.synchronize()
        assert np.allclose(dq.cpu().numpy(), O.rope(q, pos, nh, hd, theta), rtol=2e-6, atol=2e-6)
        assert np.allclose(kc[pos].cpu().numpy(), O.rope(k, pos, nkv, hd, theta), rtol=2e-6, atol=2e-6)
        assert np.array_equal(vc[pos].cpu().numpy(), v)
        assert np.array_equal(dk.cpu().numpy(), k)  # k itself is not modified


@pytest.mark.parametrize("nh,nkv,hd,T", [(32, 4, 64, 1), (32, 4, 64, 128), (32, 4, 64, 129), (32, 4, 64, 512),
                                         (32, 8, 128, 300), (8, 8, 64, 1000), (4, 1, 256, 70),
                                         (16, 8, 128, 200), (12, 6, 64, 333), (16, 4, 64, 65), (8, 8, 128, 64)])
def test_attention(L, nh, nkv, hd, T):
    say("attention", nh, nkv, hd, T)
    max_seq = 1024
    kvd = nkv * hd
    q = vec(nh * hd, T)
    kc = vec(max_seq * kvd, T + 1).reshape(max_seq, kvd)
    vc = vec(max_seq * kvd, T + 2).reshape(max_seq, kvd)
    out = torch.full((nh * hd,), float("nan"), device="cuda")
    dpos = torch.tensor([T - 1], dtype=torch.int32, device="cuda")
    dq, dk, dv = dev(q), dev(kc), dev(vc)
    assert L.jh_attention_dev(P(dq), P(dk), P(dv), nh, nkv, hd, P(dpos), max_seq, P(out), None) == 0
    got = out.cpu().numpy()
    ref = O.gqa(q, kc, vc, nh, nkv, hd, T)
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max() + 1e-7
    if T == 1:  # softmax of one score is exactly 1: out = v of the mapped KV head
        assert np.array_equal(got.reshape(nh, hd), np.repeat(vc[0].reshape(nkv, hd), nh // nkv, axis=0))


@pytest.mark.parametrize("nh,nkv,hd,pos", [(32, 4, 64, 0), (32, 4, 64, 63), (32, 4, 64, 64), (32, 4, 64, 511),
                                           (32, 8, 128, 200), (4, 1, 256, 70), (16, 8, 64, 65), (8, 8, 128, 511),
                                           (16, 8, 128, 127)])
def test_rope_attention_fused(L, nh, nkv, hd, pos):
    """rope of q and k, KV append and gqa in one call == the oracle's three steps."""
    say("rope_attention", nh, nkv, hd, pos)
    max_seq, theta, kvd = 600, 10000.0, nkv * hd
    q, k, v = vec(nh * hd, pos + 1), vec(kvd, pos + 2), vec(kvd, pos + 3)
    kc = vec(max_seq * kvd, pos + 4).reshape(max_seq, kvd)
    vc = vec(max_seq * kvd, pos + 5).reshape(max_seq, kvd)
    dkc, dvc, dq, dk, dv = dev(kc), dev(vc), dev(q), dev(k), dev(v)  # alive across the call
    out = torch.full((nh * hd,), float("nan"), device="cuda")
    dpos = torch.tensor([pos], dtype=torch.int32, device="cuda")
    assert L.jh_rope_attention_dev(P(dq), P(dk), P(dv), nh, nkv, hd, P(dpos), max_seq, theta, P(dkc), P(dvc),
                                   P(out), None) == 0
    kc_ref, vc_ref = kc.copy(), vc.copy()
    kc_ref[pos] = O.rope(k, pos, nkv, hd, theta)
    vc_ref[pos] = v
    ref = O.gqa(O.rope(q, pos, nh, hd, theta), kc_ref, vc_ref, nh, nkv, hd, pos + 1)
    got = out.cpu().numpy()
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max() + 1e-7
    assert np.allclose(dkc[pos].cpu().numpy(), kc_ref[pos], rtol=2e-6, atol=2e-6)
    assert np.array_equal(dvc[pos].cpu().numpy(), v)
    assert np.array_equal(np.delete(dkc.cpu().numpy(), pos, 0), np.delete(kc, pos, 0))
    assert np.array_equal(dq.cpu().numpy(), q)  # q itself is not modified


@pytest.mark.parametrize("nh,nkv,hd", [(32, 4, 64), (32, 8, 128), (16, 8, 128), (8, 8, 64)])
@pytest.mark.parametrize("batch", [2, 8, 12])
def test_rope_attention_batched(L, nh, nkv, hd, batch):
    """jh_rope_attention_batched_dev: each request at its own position and cache
    slot (slots permuted) == the oracle's rope + append + gqa per request.
    Batches of 8 and more at head_dim 128 read V from the cache instead of LDS."""
    say("rope_attention_batched", nh, nkv, hd, batch)
    max_seq, theta, kvd, n_slots = 300, 500000.0, nkv * hd, batch + 3
    rng = np.random.default_rng(batch * 7 + hd)
    pos = rng.integers(0, max_seq, batch)
    pos[0], pos[-1] = 0, max_seq - 1
    slots = rng.permutation(n_slots)[:batch]
    q = vec(batch * nh * hd, 11 + batch).reshape(batch, nh * hd)
    k = vec(batch * kvd, 12 + batch).reshape(batch, kvd)
    v = vec(batch * kvd, 13 + batch).reshape(batch, kvd)
    kc = vec(n_slots * max_seq * kvd, 14 + batch).reshape(n_slots, max_seq, kvd)
    vc = vec(n_slots * max_seq * kvd, 15 + batch).reshape(n_slots, max_seq, kvd)
    dkc, dvc = dev(kc), dev(vc)
    out = torch.full((batch, nh * hd), float("nan"), device="cuda")
    dpos, dslot = dev(pos, torch.int32), dev(slots, torch.int32)
    dq, dk, dv = dev(q), dev(k), dev(v)  # alive across the call
    assert L.jh_rope_attention_batched_dev(P(dq), P(dk), P(dv), batch, nh, nkv, hd, P(dpos), P(dslot),
                                           n_slots, max_seq, theta, P(dkc), P(dvc), P(out), None) == 0
    got = out.cpu().numpy()
    for z in range(batch):
        p, sl = int(pos[z]), int(slots[z])
        kc_ref, vc_ref = kc[sl].copy(), vc[sl].copy()
        kc_ref[p] = O.rope(k[z], p, nkv, hd, theta)
        vc_ref[p] = v[z]
        ref = O.gqa(O.rope(q[z], p, nh, hd, theta), kc_ref, vc_ref, nh, nkv, hd, p + 1)
        assert np.abs(got[z] - ref).max() <= 1e-5 * np.abs(ref).max() + 1e-7, z
        assert np.array_equal(dvc[sl, p].cpu().numpy(), v[z])


def test_attention_arguments(L):
    d = torch.zeros(64, device="cuda")
    pos = torch.zeros(1, dtype=torch.int32, device="cuda")
    assert L.jh_attention_dev(P(d), P(d), P(d), 6, 4, 64, P(pos), 8, P(d), None) != 0  # 6 % 4
    assert L.jh_attention_dev(P(d), P(d), P(d), 4, 4, 63, P(pos), 8, P(d), None) != 0  # odd head_dim
    assert L.jh_attention_dev(P(d), P(d), P(d), 4, 4, 64, None, 8, P(d), None) != 0


def test_silu_mul_and_pos_increment(L):
    n = 5632
    g, u = vec(n, 7, 4.0), vec(n, 8)
    out = torch.empty(n, device="cuda")
    dg, du = dev(g), dev(u)  # alive across the call
    assert L.jh_silu_mul_dev(P(dg), P(du), n, P(out), None) == 0
    assert np.allclose(out.cpu().numpy(), O.silu_mul(g, u), rtol=2e-6, atol=1e-7)
    pos = torch.tensor([41], dtype=torch.int32, device="cuda")
    assert L.jh_pos_increment_dev(P(pos), 1, None) == 0
    assert int(pos.item()) == 42


# ------------------------------------------------------------------ whole steps vs the oracle

def packed_model(cfg, seed):
    """Random weights drawn and quantized on the device (the device quantizer is
    bit-exact with the oracle's), with host copies of every tensor for the oracle."""
    w = D.LlamaWeights.random(cfg, seed=seed)
    layers = []
    for lw in w.layers:
        d = {"attn_norm": lw.attn_norm.cpu().numpy(), "ffn_norm": lw.ffn_norm.cpu().numpy()}
        for m, mat in lw.mats.items():
            d["w" + m], d["type_" + m] = mat.packed_bytes(), mat.type
        layers.append(d)
    return w, layers, w.output_norm.cpu().numpy(), w.output.packed_bytes()


def oracle_step(cfg, layers, out_norm, out_raw, x, pos, kc, vc):
    """The oracle's logits and the normed final x the output projection took."""
    dims = dict(hidden=cfg.hidden_dim, n_heads=cfg.num_heads, n_kv_heads=cfg.num_kv_heads, head_dim=cfg.head_dim,
                ffn=cfg.intermediate_size, eps=cfg.rms_norm_eps, theta=cfg.rope_theta)
    for li, lw in enumerate(layers):
        x = O.llama_layer(lw, dims, x, pos, kc[li], vc[li])
    xn = O.rmsnorm(x, out_norm, cfg.rms_norm_eps)
    return O.matvec(D.Q4_K_M["output"], out_raw, xn, 0, cfg.vocab_size, cfg.hidden_dim), xn


def check_logits(cfg, got, ref_xn, out_raw, what):
    """The GEMV bar per logit row: |got - ref| / max(|ref|, 1e-3 * sum_c |w_rc xn_c|) <= 1e-3,
    with the oracle's output weights and normed final x (errors of every layer included)."""
    ref, xn = ref_xn
    deq = O.dequantize(D.Q4_K_M["output"], out_raw, cfg.vocab_size, cfg.hidden_dim).astype(np.float64)
    scale = np.abs(deq.reshape(cfg.vocab_size, cfg.hidden_dim)) @ np.abs(xn.astype(np.float64))
    ref = ref.astype(np.float64)
    err = np.abs(got.astype(np.float64) - ref)
    rel = float((err / np.maximum(np.abs(ref), 1e-3 * scale)).max())
    say(what, f"max per-row rel-err {rel:.2e} (max err / max|logit| {err.max() / np.abs(ref).max():.2e})")
    assert rel <= 1e-3, (what, rel)


def test_decode_steps_small_model():
    cfg = D.LlamaConfig(hidden_dim=256, num_layers=2, num_heads=4, num_kv_heads=2, head_dim=64,
                        intermediate_size=512, vocab_size=1000)
    layers, out_norm, out_raw = packed_model(cfg, 11)[1:]
    # upload path: the same packed bytes through jh_qmat_upload
    w = D.LlamaWeights.from_packed(cfg, layers, out_norm, out_raw, D.Q4_K_M["output"])
    dec = D.LlamaDecoder(w, max_seq=64)
    kc = np.zeros((cfg.num_layers, 64, cfg.kv_dim), np.float32)
    vc = np.zeros_like(kc)
    for pos in range(5):
        x = vec(cfg.hidden_dim, 100 + pos)
        say("small step", pos)
        got = dec.forward(x, pos)
        ref = oracle_step(cfg, layers, out_norm, out_raw, x, pos, kc, vc)
        check_logits(cfg, got, ref, out_raw, f"pos {pos}")
        k_dev = dec.k_cache[:, : pos + 1].cpu().numpy()
        assert np.allclose(k_dev, kc[:, : pos + 1], rtol=1e-3, atol=1e-3 * np.abs(kc).max())
    with pytest.raises(IllegalArgumentException):
        dec.forward(np.zeros(7, np.float32), 0)
    w.close()


def test_decode_graph_replay_matches_eager():
    cfg = D.LlamaConfig(hidden_dim=256, num_layers=2, num_heads=4, num_kv_heads=2, head_dim=64,
                        intermediate_size=512, vocab_size=1000)
    w = packed_model(cfg, 12)[0]
    eager = D.LlamaDecoder(w, max_seq=32)
    graph = D.LlamaDecoder(w, max_seq=32)
    s = torch.cuda.Stream()
    g = graph.capture(s)   # its warm-up step wrote position 0; the replays rewrite it
    graph.pos.fill_(0)
    for pos in range(4):
        x = vec(cfg.hidden_dim, 200 + pos)
        say("graph step", pos)
        ref = eager.forward(x, pos)
        with torch.cuda.stream(s):
            graph.x.copy_(torch.from_numpy(x))
            g.replay()
        s.synchronize()
        torch.cuda.synchronize()
        assert np.array_equal(graph.logits.cpu().numpy(), ref), pos
        assert int(graph.pos.item()) == pos + 1
    w.close()


def test_decode_tinyllama_shape_prefilled_cache():
    """TinyLlama-1.1B shape (22 layers, hidden 2048, 32 / 4 heads, FFN 5632,
    vocab 32000, Q4_K_M) at position 511 with the KV cache pre-filled with N(0, 1)."""
    cfg = D.LlamaConfig(hidden_dim=2048, num_layers=22, num_heads=32, num_kv_heads=4, head_dim=64,
                        intermediate_size=5632, vocab_size=32000)
    say("tinyllama: quantizing")
    w, layers, out_norm, out_raw = packed_model(cfg, 13)
    dec = D.LlamaDecoder(w, max_seq=512)
    kc = vec(cfg.num_layers * 512 * cfg.kv_dim, 14).reshape(cfg.num_layers, 512, cfg.kv_dim)
    vc = vec(cfg.num_layers * 512 * cfg.kv_dim, 15).reshape(cfg.num_layers, 512, cfg.kv_dim)
    dec.k_cache.copy_(torch.from_numpy(kc))
    dec.v_cache.copy_(torch.from_numpy(vc))
    x = vec(cfg.hidden_dim, 16)
    say("tinyllama: step")
    got = dec.forward(x, 511)
    ref = oracle_step(cfg, layers, out_norm, out_raw, x, 511, kc, vc)
    check_logits(cfg, got, ref, out_raw, "tinyllama pos 511")
    w.close()
