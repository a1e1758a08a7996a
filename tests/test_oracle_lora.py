"""LoRA overlay on the CPU: the oracle's LoraAdapter.forward restatement
(lora/src/main/java/cab/ml/juno/lora/LoraAdapter.java:79-98) pinned by the
reference's own checks (zero B gives a zero delta, LoraAdapterTest.java:65-71;
the delta scales with alpha, :185-197), float64 brute force and a rank-1 closed
form; and the reference's checkpoint format (LoraAdapterSet.java:68-124)
read and written by juno_amd.lora.
"""
import struct

import numpy as np
import pytest

import oracle as O
from juno_amd import IOException
from juno_amd.lora import LoraAdapter, LoraAdapterSet


def rnd(n, seed, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(n) * scale).astype(np.float32)


def test_zero_b_gives_zero_delta():  # LoraAdapterTest.java:65-71
    d = O.lora_forward(rnd(8 * 16, 1), np.zeros(32 * 8, np.float32), 8, 16, 32, 2.0, rnd(16, 2))
    assert np.all(d == 0.0)


def test_delta_scales_with_alpha():  # LoraAdapterTest.java:185-197
    a, b, x = rnd(4 * 64, 3), rnd(48 * 4, 4), rnd(64, 5)
    d1 = O.lora_forward(a, b, 4, 64, 48, 1.5, x)
    d2 = O.lora_forward(a, b, 4, 64, 48, 3.0, x)
    assert np.array_equal(d2, 2 * d1)  # the scale multiplies last: doubling it is exact


def test_matches_float64():
    for rank, n_in, n_out, seed in [(1, 7, 3, 0), (8, 2048, 256, 1), (64, 4096, 1024, 2)]:
        a, b, x = rnd(rank * n_in, seed, 0.02), rnd(n_out * rank, seed + 1), rnd(n_in, seed + 2)
        ref = (b.astype(np.float64).reshape(n_out, rank) @ (a.astype(np.float64).reshape(rank, n_in) @ x)) * 0.5
        got = O.lora_forward(a, b, rank, n_in, n_out, 0.5, x)
        bound = 1e-5 * (np.abs(b.reshape(n_out, rank)) @ (np.abs(a.reshape(rank, n_in)) @ np.abs(x))) * 0.5
        assert np.all(np.abs(got - ref) <= bound + 1e-12)


def test_rank1_unit_a_picks_one_input():
    n_in, n_out, i = 10, 6, 7
    a = np.zeros(n_in, np.float32)
    a[i] = 1.0
    b, x = rnd(n_out, 9), rnd(n_in, 10)
    assert np.array_equal(O.lora_forward(a, b, 1, n_in, n_out, 2.0, x), (b * x[i]) * np.float32(2.0))


def reference_checkpoint(entries):
    """Bytes in LoraAdapterSet.save's layout (LoraAdapterSet.java:68-89)."""
    out = struct.pack(">iii", 0x4C4F5241, 1, len(entries))
    for key, rank, n_in, n_out, alpha, a, b in entries:
        kb = key.encode()
        out += struct.pack(">i", len(kb)) + kb + struct.pack(">iiif", rank, n_in, n_out, alpha)
        out += np.asarray(a, ">f4").tobytes() + np.asarray(b, ">f4").tobytes()
    return out


def test_checkpoint_load_and_save_round_trip(tmp_path):
    a0, b0, a1, b1 = rnd(4 * 32, 1), rnd(16 * 4, 2), rnd(8 * 32, 3), rnd(32 * 8, 4)
    p = tmp_path / "adapters.lora"
    p.write_bytes(reference_checkpoint([("0:wq", 4, 32, 16, 8.0, a0, b0), ("3:wv", 8, 32, 32, 4.0, a1, b1)]))
    s = LoraAdapterSet.load(p)
    assert s.size() == 2 and s.get(1, "wq") is None
    q, v = s.get(0, "wq"), s.get(3, "wv")
    assert (q.rank, q.in_dim, q.out_dim, q.scale) == (4, 32, 16, 2.0)
    assert (v.rank, v.in_dim, v.out_dim, v.scale) == (8, 32, 32, 0.5)
    assert np.array_equal(q.a_host, a0) and np.array_equal(v.b_host, b1)
    p2 = tmp_path / "again.lora"
    s.save(p2)
    assert p2.read_bytes() == p.read_bytes()


def test_checkpoint_errors(tmp_path):
    p = tmp_path / "bad.lora"
    p.write_bytes(struct.pack(">iii", 0x12345678, 1, 0))
    with pytest.raises(IOException, match="Not a LoRA checkpoint"):
        LoraAdapterSet.load(p)
    p.write_bytes(struct.pack(">iii", 0x4C4F5241, 2, 0))
    with pytest.raises(IOException, match="Unsupported LoRA checkpoint version: 2"):
        LoraAdapterSet.load(p)
    p.write_bytes(reference_checkpoint([("0:wq", 4, 32, 16, 8.0, rnd(128, 1), rnd(64, 2))])[:-4])
    with pytest.raises(IOException, match="truncated"):
        LoraAdapterSet.load(p)
    with pytest.raises(Exception, match="rank must be >= 1"):
        LoraAdapter(0, 4, 4, 1.0, [], [])
