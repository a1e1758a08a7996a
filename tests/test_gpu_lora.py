"""LoRA overlay on the device (jh_lora_apply_dev through juno_amd.lora) against
the oracle's LoraAdapter.forward (LoraAdapter.java:79-98), and decode steps
with "wq" / "wv" adapters applied after the Q and V projections
(LoraTrainableHandler.java:475-476) against a step composed from the oracle's
pieces, single-request and batched.

Tolerance: the delta within 1e-5 of sum |B| |A| |x| * scale per element (order
of fp32 sums only); logits within 1e-3 of max |logit|.
"""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from juno_amd import decode as D  # noqa: E402
from juno_amd.lora import LoraAdapter, LoraAdapterSet  # noqa: E402
from juno_amd.pipeline import LlamaBatchPipeline  # noqa: E402


def rnd(n, seed, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(n) * scale).astype(np.float32)


@pytest.mark.parametrize("rank,n_in,n_out,batch", [(1, 64, 32, 1), (8, 2048, 256, 3), (16, 4096, 4096, 32),
                                                   (64, 2048, 2048, 5)])
def test_apply_matches_oracle(rank, n_in, n_out, batch):
    a, b = rnd(rank * n_in, rank, 0.02), rnd(n_out * rank, rank + 1)
    ad = LoraAdapter.from_weights(rank, n_in, n_out, 2.0 * rank, a, b)
    X = rnd(batch * n_in, 7).reshape(batch, n_in)
    Y0 = rnd(batch * n_out, 8).reshape(batch, n_out)
    dX, dY = torch.from_numpy(X).cuda(), torch.from_numpy(Y0).cuda()
    ad.apply_dev(dX.data_ptr(), dY.data_ptr(), batch)
    torch.cuda.synchronize()
    got = dY.cpu().numpy()
    bound = 1e-5 * (np.abs(b.reshape(n_out, rank)) @ (np.abs(a.reshape(rank, n_in)) @ np.abs(X.T))).T * 2.0
    for j in range(batch):
        ref = Y0[j] + O.lora_forward(a, b, rank, n_in, n_out, ad.scale, X[j])
        assert np.all(np.abs(got[j] - ref) <= bound[j] + 1e-6 * np.abs(Y0[j])), j
    assert np.allclose(ad.forward(X[0]), O.lora_forward(a, b, rank, n_in, n_out, ad.scale, X[0]), rtol=1e-4,
                       atol=1e-5 * np.abs(got).max())


def test_zero_b_leaves_outputs_unchanged():
    ad = LoraAdapter.from_weights(8, 512, 128, 16.0, rnd(8 * 512, 1), np.zeros(128 * 8, np.float32))
    y = torch.from_numpy(rnd(128, 2)).cuda()
    y0 = y.clone()
    x = torch.from_numpy(rnd(512, 3)).cuda()
    ad.apply_dev(x.data_ptr(), y.data_ptr(), 1)
    torch.cuda.synchronize()
    assert torch.equal(y, y0)


CFG = D.LlamaConfig(hidden_dim=256, num_layers=2, num_heads=4, num_kv_heads=2, head_dim=64, intermediate_size=512,
                    vocab_size=1000)


def make_lora(cfg):
    s = LoraAdapterSet()
    for li in range(cfg.num_layers):
        s.add(li, "wq", LoraAdapter.from_weights(8, cfg.hidden_dim, cfg.hidden_dim, 16.0,
                                                 rnd(8 * cfg.hidden_dim, 10 + li, 0.05), rnd(cfg.hidden_dim * 8, 20 + li, 0.05)))
        s.add(li, "wv", LoraAdapter.from_weights(4, cfg.hidden_dim, cfg.kv_dim, 4.0,
                                                 rnd(4 * cfg.hidden_dim, 30 + li, 0.05), rnd(cfg.kv_dim * 4, 40 + li, 0.05)))
    return s


def oracle_step_lora(cfg, w, lora, x, pos, kc, vc):
    """transformerLayer with the LoRA deltas (LoraTrainableHandler.inferenceLayer, :464-487)
    composed from the oracle's pieces."""
    H, nh, nkv, hd, eps = cfg.hidden_dim, cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.rms_norm_eps
    mv = lambda m, v: O.matvec(m.type, m.packed_bytes(), v, 0, m.rows, m.cols)
    for li, lw in enumerate(w.layers):
        xn = O.rmsnorm(x, lw.attn_norm.cpu().numpy(), eps)
        m = lw.mats
        q, k, v = mv(m["q"], xn), mv(m["k"], xn), mv(m["v"], xn)
        for proj, out in (("wq", q), ("wv", v)):
            ad = lora.get(li, proj)
            out += O.lora_forward(ad.a_host, ad.b_host, ad.rank, ad.in_dim, ad.out_dim, ad.scale, xn)
        q = O.rope(q, pos, nh, hd, cfg.rope_theta)
        k = O.rope(k, pos, nkv, hd, cfg.rope_theta)
        kc[li][pos], vc[li][pos] = k, v
        att = O.gqa(q, kc[li], vc[li], nh, nkv, hd, pos + 1)
        x2 = O.add(x, mv(m["o"], att))
        xn2 = O.rmsnorm(x2, lw.ffn_norm.cpu().numpy(), eps)
        ffn = mv(m["down"], O.silu_mul(mv(m["gate"], xn2), mv(m["up"], xn2)))
        x = O.add(x2, ffn)
    return O.matvec(w.output.type, w.output.packed_bytes(), O.rmsnorm(x, w.output_norm.cpu().numpy(), eps), 0,
                    cfg.vocab_size, cfg.hidden_dim)


def err(a, b):
    return float(np.abs(a.astype(np.float64) - b).max() / np.abs(b).max())


def test_decoder_with_lora_matches_oracle():
    w = D.LlamaWeights.random(CFG, seed=41, embeddings=True)
    lora = make_lora(CFG)
    dec = D.LlamaDecoder(w, max_seq=16, lora=lora)
    plain = D.LlamaDecoder(w, max_seq=16)
    kc = np.zeros((CFG.num_layers, 16, CFG.kv_dim), np.float32)
    vc = np.zeros_like(kc)
    for pos in range(3):
        x = rnd(CFG.hidden_dim, 50 + pos)
        got = dec.forward(x, pos)
        ref = oracle_step_lora(CFG, w, lora, x, pos, kc, vc)
        assert err(got, ref) <= 1e-3, pos
        assert err(plain.forward(x, pos), ref) > 1e-3  # the adapters change the output
    # batched: the same adapters through forwardBatch equal serial single-request decoders
    pipe = LlamaBatchPipeline(w, max_seq=8, max_batch=4, lora=lora)
    serial = [D.LlamaDecoder(w, max_seq=8, lora=lora) for _ in range(3)]
    for pos in range(2):
        toks = [[3 + pos], [500], [999 - pos]]
        got = pipe.forward_batch(["a", "b", "c"], toks, [pos] * 3)
        for dec_i, t, g in zip(serial, toks, got):
            assert err(g, dec_i.forward_token(t[-1], pos)) <= 1e-3
    w.close()
