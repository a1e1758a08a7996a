"""Pins the oracle's restatement of the decode step around the matvec
(oracle/juno_oracle_decode.c): rmsNorm, rope, softmax, gqa, silu, add and
their composition into transformerLayer (LlamaTransformerHandler.java:743-800).

Checks are the reference's own known answers where it has them (rope at
position 0 is the identity and forward-then-inverse returns the input,
LoraTrainableHandlerTest.java:249-276) and otherwise closed forms and float64
brute force chosen so that a dropped term, a wrong sign or index, or a
misordered step fails.
"""
import numpy as np
import pytest

import oracle as O

RNG = np.random.default_rng(1234)


def vec(n, seed, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(n) * scale).astype(np.float32)


# ------------------------------------------------------------------ rmsNorm

def test_rmsnorm_matches_float64_formula():
    for n, seed in [(8, 1), (2048, 2), (4096, 3)]:
        x, w = vec(n, seed), vec(n, seed + 100)
        eps = 1e-5
        ref = w.astype(np.float64) * x / np.sqrt(np.mean(x.astype(np.float64) ** 2) + eps)
        got = O.rmsnorm(x, w, eps)
        assert np.allclose(got, ref, rtol=2e-5, atol=1e-6)


def test_rmsnorm_unit_weights_give_unit_rms_and_scale_invariance():
    x = vec(1024, 5) * 7.0
    y = O.rmsnorm(x, np.ones(1024, np.float32), 0.0)
    assert abs(np.sqrt(np.mean(y.astype(np.float64) ** 2)) - 1.0) < 1e-5
    assert np.allclose(O.rmsnorm(3.0 * x, np.ones(1024, np.float32), 0.0), y, rtol=1e-5, atol=1e-6)
    # eps enters inside the square root: a zero vector stays finite (zero)
    assert np.all(O.rmsnorm(np.zeros(16, np.float32), np.ones(16, np.float32), 1e-5) == 0)


# ------------------------------------------------------------------ rope

def test_rope_position_zero_is_identity():  # LoraTrainableHandlerTest.java:268-275
    x = vec(2 * 8, 50)
    assert np.array_equal(O.rope(x, 0, 2, 8, 10000.0), x)


def test_rope_forward_then_inverse_round_trip():  # LoraTrainableHandlerTest.java:251-263
    x = vec(4 * 8, 40)
    y = O.rope(O.rope(x, 7, 4, 8, 10000.0), -7, 4, 8, 10000.0)  # angle -pos*freq rotates back
    assert np.allclose(y, x, atol=1e-5)


def test_rope_is_complex_rotation_of_adjacent_pairs():
    n_heads, hd, theta = 4, 64, 10000.0
    x = vec(n_heads * hd, 60)
    for pos in (1, 17, 511):
        got = O.rope(x, pos, n_heads, hd, theta).astype(np.float64).reshape(n_heads, hd // 2, 2)
        z = x.astype(np.float64).reshape(n_heads, hd // 2, 2)
        zc = z[..., 0] + 1j * z[..., 1]
        i = np.arange(hd // 2)
        ref = zc * np.exp(1j * pos / theta ** (2.0 * i / hd))
        assert np.allclose(got[..., 0], ref.real, atol=2e-5)
        assert np.allclose(got[..., 1], ref.imag, atol=2e-5)
        # a split-half pairing (x[i], x[i + hd/2]) would not preserve these norms
        assert np.allclose(np.hypot(got[..., 0], got[..., 1]), np.abs(zc), rtol=1e-5)


# ------------------------------------------------------------------ softmax / gqa

def test_softmax_invariants():
    s = vec(37, 70, 3.0)
    p = O.softmax(s)
    assert abs(p.astype(np.float64).sum() - 1.0) < 1e-6
    ref = np.exp(s.astype(np.float64) - s.max())
    assert np.allclose(p, ref / ref.sum(), rtol=1e-5)
    assert np.allclose(O.softmax(s + 100.0), p, rtol=1e-5)
    assert np.allclose(O.softmax(np.full(8, 2.5, np.float32)), 0.125)


def gqa_f64(q, kc, vc, nh, nkv, hd, T):
    q = q.astype(np.float64).reshape(nh, hd)
    k = kc[:T].astype(np.float64).reshape(T, nkv, hd)
    v = vc[:T].astype(np.float64).reshape(T, nkv, hd)
    out = np.zeros((nh, hd))
    for h in range(nh):
        g = h // (nh // nkv)
        s = k[:, g, :] @ q[h] / np.sqrt(hd)
        p = np.exp(s - s.max())
        p /= p.sum()
        out[h] = p @ v[:, g, :]
    return out.reshape(-1)


def test_gqa_single_position_returns_v_of_the_mapped_head():
    nh, nkv, hd = 8, 2, 16
    q = vec(nh * hd, 80)
    kc, vc = vec(nkv * hd, 81).reshape(1, -1), vec(nkv * hd, 82).reshape(1, -1)
    out = O.gqa(q, kc, vc, nh, nkv, hd, 1).reshape(nh, hd)
    for h in range(nh):
        assert np.array_equal(out[h], vc[0].reshape(nkv, hd)[h // (nh // nkv)])


def test_gqa_matches_float64_brute_force():
    for nh, nkv, hd, T in [(8, 2, 16, 5), (32, 4, 64, 512), (32, 8, 128, 33)]:
        q = vec(nh * hd, 90 + T)
        kc = vec(T * nkv * hd, 91 + T).reshape(T, -1)
        vc = vec(T * nkv * hd, 92 + T).reshape(T, -1)
        got = O.gqa(q, kc, vc, nh, nkv, hd, T)
        assert np.allclose(got, gqa_f64(q, kc, vc, nh, nkv, hd, T), rtol=1e-4, atol=2e-6)


def test_gqa_equal_keys_average_the_values():
    nh, nkv, hd, T = 4, 1, 8, 6
    q = vec(nh * hd, 95)
    kc = np.tile(vec(hd, 96), (T, 1))
    vc = vec(T * hd, 97).reshape(T, hd)
    out = O.gqa(q, kc, vc, nh, nkv, hd, T).reshape(nh, hd)
    assert np.allclose(out, vc.mean(axis=0), atol=1e-6)


# ------------------------------------------------------------------ silu / add

def test_silu_and_swiglu():
    x = vec(1000, 100, 4.0)
    ref = x.astype(np.float64) / (1.0 + np.exp(-x.astype(np.float64)))
    got = np.array([O.silu(float(v)) for v in x[:50]])
    assert np.allclose(got, ref[:50], rtol=1e-6, atol=1e-7)
    assert O.silu(0.0) == 0.0
    u = vec(1000, 101)
    assert np.allclose(O.silu_mul(x, u), (ref * u).astype(np.float32), rtol=1e-5, atol=1e-7)
    assert np.array_equal(O.add(x, u), x + u)


# ------------------------------------------------------------------ transformerLayer composition

def make_layer(dims, seed, types=None):
    """Random N(0, 0.02) weights quantized with the oracle's quantizers."""
    H, I = dims["hidden"], dims["ffn"]
    KV = dims["n_kv_heads"] * dims["head_dim"]
    shapes = {"q": (H, H), "k": (KV, H), "v": (KV, H), "o": (H, H), "gate": (I, H), "up": (I, H), "down": (H, I)}
    types = types or {"q": O.Q4_K, "k": O.Q4_K, "v": O.Q6_K, "o": O.Q4_K, "gate": O.Q4_K, "up": O.Q4_K,
                      "down": O.Q6_K}
    rng = np.random.default_rng(seed)
    layer = {"attn_norm": (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32),
             "ffn_norm": (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)}
    for m, (r, c) in shapes.items():
        layer["w" + m] = O.quantize(types[m], (rng.standard_normal(r * c) * 0.02).astype(np.float32))
        layer["type_" + m] = types[m]
        layer["shape_" + m] = (r, c)
    return layer


def layer_f64(layer, dims, x, pos, kc, vc):
    """float64 statement of transformerLayer from the oracle's dequantized weights."""
    H, nh, nkv, hd, eps, theta = (dims[k] for k in ("hidden", "n_heads", "n_kv_heads", "head_dim", "eps", "theta"))
    W = {m: O.dequantize(layer["type_" + m], layer["w" + m], *layer["shape_" + m]).astype(np.float64)
         for m in ("q", "k", "v", "o", "gate", "up", "down")}
    def rms(v, w):
        return w * v / np.sqrt(np.mean(v * v) + eps)
    def rot(v, nheads):
        z = v.reshape(nheads, hd // 2, 2)
        zc = (z[..., 0] + 1j * z[..., 1]) * np.exp(1j * pos / theta ** (2.0 * np.arange(hd // 2) / hd))
        return np.stack([zc.real, zc.imag], -1).reshape(-1)
    x = x.astype(np.float64)
    xn = rms(x, layer["attn_norm"].astype(np.float64))
    q, k, v = rot(W["q"] @ xn, nh), rot(W["k"] @ xn, nkv), W["v"] @ xn
    kc = kc.astype(np.float64).copy()
    vc = vc.astype(np.float64).copy()
    kc[pos], vc[pos] = k, v
    att = gqa_f64(q, kc, vc, nh, nkv, hd, pos + 1)
    x2 = x + W["o"] @ att
    xn2 = rms(x2, layer["ffn_norm"].astype(np.float64))
    g, u = W["gate"] @ xn2, W["up"] @ xn2
    return x2 + W["down"] @ (g / (1 + np.exp(-g)) * u), k, v


@pytest.mark.parametrize("pos", [0, 5, 63])
def test_llama_layer_matches_float64_composition(pos):
    dims = dict(hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, eps=1e-5, theta=10000.0)
    layer = make_layer(dims, 7)
    KV = dims["n_kv_heads"] * dims["head_dim"]
    kc = np.ascontiguousarray(vec(64 * KV, 8).reshape(64, KV))
    vc = np.ascontiguousarray(vec(64 * KV, 9).reshape(64, KV))
    x = vec(256, 10)
    ref, k_ref, v_ref = layer_f64(layer, dims, x, pos, kc, vc)
    kc_o, vc_o = kc.copy(), vc.copy()
    y = O.llama_layer(layer, dims, x, pos, kc_o, vc_o)
    assert np.allclose(kc_o[pos], k_ref, rtol=1e-4, atol=1e-5)
    assert np.allclose(vc_o[pos], v_ref, rtol=1e-4, atol=1e-5)
    assert np.array_equal(np.delete(kc_o, pos, 0), np.delete(kc, pos, 0))  # other positions untouched
    assert np.allclose(y, ref, rtol=1e-4, atol=1e-4 * np.abs(ref).max())
