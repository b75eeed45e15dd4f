"""Pins of the token-pipeline and embedding oracle (CPU only).

batch_at is checked against the reference's own test vector
(tests/test_baseline.py:30-38 of the reference) and its test stream
(arange(4097) % 31, tests/test_optimized.py:89); the embedding forward against
numpy's gather and broadcast add; the backward against np.add.at / numpy sums
on small-integer gradients, where every summation order gives the same exact
result, and against fp64 sums for random gradients.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle


def test_batch_at_reference_vector(tmp_path):
    path = tmp_path / "tokens.bin"
    data = np.memmap(path, dtype=np.uint16, mode="w+", shape=(12,))
    data[:] = np.arange(12)
    data.flush()
    x, y, count = oracle.batch_at(data, cursor=0, batch_size=2, sequence_length=8, target_limit=11)
    assert count == 11
    assert x.shape == y.shape == (2, 8)
    assert int((y != -100).sum()) == 11
    assert y.flatten()[:11].tolist() == list(range(1, 12))
    assert x.flatten()[:11].tolist() == list(range(0, 11))
    assert x.flatten()[11:].tolist() == [0] * 5
    assert y.flatten()[11:].tolist() == [-100] * 5
    assert x.dtype == y.dtype == np.int64


def test_batch_at_stream_shift_identity():
    stream = (np.arange(4097) % 31).astype(np.uint16)
    cursor = 0
    seen = 0
    while True:
        try:
            x, y, count = oracle.batch_at(stream, cursor, 3, 128, 4096)
        except StopIteration:
            break
        fx, fy = x.flatten(), y.flatten()
        assert np.array_equal(fx[1:count], fy[:count - 1])
        assert np.array_equal(fy[:count], (np.arange(cursor + 1, cursor + count + 1) % 31))
        assert count == min(3 * 128, 4096 - cursor)
        cursor += count
        seen += count
    assert seen == 4096
    with pytest.raises(StopIteration):
        oracle.batch_at(stream, 4096, 3, 128, 4096)


def test_batch_at_large_ids_keep_uint16_range():
    stream = np.array([65535, 50256, 0, 1, 65534], np.uint16)
    x, y, count = oracle.batch_at(stream, 0, 1, 4, 4)
    assert x.tolist() == [[65535, 50256, 0, 1]] and y.tolist() == [[50256, 0, 1, 65534]]


def tables(vocab, max_seq, d, seed=0):
    g = np.random.default_rng(seed)
    return (g.standard_normal((vocab, d)).astype(np.float32),
            g.standard_normal((max_seq, d)).astype(np.float32))


def test_embed_fwd_is_gather_plus_broadcast():
    tok, pos = tables(101, 16, 32)
    ids = np.random.default_rng(1).integers(0, 101, (3, 12))
    out = oracle.embed_fwd(ids, tok, pos)
    ref = tok[ids] + pos[None, :12]
    assert np.array_equal(out, ref)


def test_embed_fwd_bad_ids_are_nan_rows():
    tok, pos = tables(10, 4, 8)
    ids = np.array([[0, 10, -1, 9]])
    out = oracle.embed_fwd(ids, tok, pos)
    assert np.isnan(out[0, 1]).all() and np.isnan(out[0, 2]).all()
    assert np.array_equal(out[0, 0], tok[0] + pos[0]) and np.array_equal(out[0, 3], tok[9] + pos[3])


def zipf_ids(rng, shape, vocab):
    # a few very frequent ids (runs crossing many blocks) over a uniform tail
    ids = rng.integers(0, vocab, shape)
    hot = rng.random(shape) < 0.4
    ids[hot] = rng.integers(0, 3, int(hot.sum()))
    return ids


@pytest.mark.parametrize("block", [1, 3, 16, 1000])
def test_embed_bwd_integer_grads_exact(block):
    rng = np.random.default_rng(2)
    vocab, max_seq, d, batch, seq = 50, 40, 12, 5, 33
    ids = zipf_ids(rng, (batch, seq), vocab)
    dout = rng.integers(-8, 9, (batch, seq, d)).astype(np.float32)
    dtok, dpos = oracle.embed_bwd(ids, dout, vocab, max_seq, block=block)
    ref_tok = np.zeros((vocab, d), np.float32)
    np.add.at(ref_tok, ids.reshape(-1), dout.reshape(-1, d))
    assert np.array_equal(dtok, ref_tok)
    ref_pos = np.zeros((max_seq, d), np.float32)
    ref_pos[:seq] = dout.sum(0)
    assert np.array_equal(dpos, ref_pos)


def test_embed_bwd_accumulates_and_skips_bad_ids():
    rng = np.random.default_rng(3)
    vocab, max_seq, d = 20, 8, 4
    ids = np.array([[0, 5, 20, -3, 5, 5, 19, 0]])
    dout = rng.integers(-4, 5, (1, 8, d)).astype(np.float32)
    base_tok = rng.integers(-4, 5, (vocab, d)).astype(np.float32)
    base_pos = rng.integers(-4, 5, (max_seq, d)).astype(np.float32)
    dtok, dpos = oracle.embed_bwd(ids, dout, vocab, max_seq, dtok=base_tok.copy(), dpos=base_pos.copy())
    ref_tok = base_tok.copy()
    ok = (ids >= 0) & (ids < vocab)
    np.add.at(ref_tok, ids[ok], dout[ok])
    assert np.array_equal(dtok, ref_tok)
    assert np.array_equal(dpos, base_pos + dout[0])


def test_embed_bwd_float_grads_match_fp64():
    rng = np.random.default_rng(4)
    vocab, max_seq, d, batch, seq = 300, 64, 20, 7, 64
    ids = zipf_ids(rng, (batch, seq), vocab)
    dout = rng.standard_normal((batch, seq, d)).astype(np.float32)
    dtok, dpos = oracle.embed_bwd(ids, dout, vocab, max_seq)
    ref_tok = np.zeros((vocab, d))
    np.add.at(ref_tok, ids.reshape(-1), dout.reshape(-1, d).astype(np.float64))
    counts = np.bincount(ids.reshape(-1), minlength=vocab)[:, None]
    abs_sum = np.zeros((vocab, d))
    np.add.at(abs_sum, ids.reshape(-1), np.abs(dout.reshape(-1, d)).astype(np.float64))
    assert (np.abs(dtok - ref_tok) <= counts * 2.0 ** -24 * abs_sum + 1e-30).all()
    ref_pos = dout.astype(np.float64).sum(0)
    assert np.allclose(dpos[:seq], ref_pos, rtol=0, atol=batch * 2.0 ** -24 * np.abs(dout).sum(0).max())
    assert (dpos[seq:] == 0).all()


def test_embed_bwd_block_order_only_matters_across_blocks():
    # every run inside one block: the result is the plain sequential sum for
    # any block size that keeps runs whole
    rng = np.random.default_rng(5)
    ids = np.repeat(np.arange(8), 4)[None, :]      # runs of 4 in sorted order
    dout = rng.standard_normal((1, 32, 6)).astype(np.float32)
    a, _ = oracle.embed_bwd(ids, dout, 8, 32, block=4)
    b, _ = oracle.embed_bwd(ids, dout, 8, 32, block=32)
    seq = np.zeros((8, 6), np.float32)
    for v in range(8):
        acc = np.zeros(6, np.float32)
        for i in range(32):
            if ids[0, i] == v:
                acc = acc + dout[0, i]
        seq[v] = acc
    assert np.array_equal(a, seq) and np.array_equal(b, seq)
