"""GPU parity of the token pipeline and the fused token + position embedding.

``batch_at`` must reproduce the oracle's restatement of
scripts/train_baseline.py:50-63 bit for bit (integers), from a host uint16
memmap and from a stream resident in HBM.  The embedding forward is one fp32
add per element and must match the oracle bit for bit; the backward sums in a
fixed order the oracle restates (stable id sort, blocks of 16 sorted entries),
so it must match bit for bit too, and match torch's nn.Embedding autograd
within the fp32 summation bound.  Id streams include a heavy head (runs that
cross many blocks), a single id repeated over every token, and ids outside
the vocabulary.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from reversability_amd import data, embedding

pytestmark = pytest.mark.gpu


def test_batch_at_reference_vector(cuda_device, tmp_path):
    path = tmp_path / "tokens.bin"
    stream = np.memmap(path, dtype=np.uint16, mode="w+", shape=(12,))
    stream[:] = np.arange(12)
    stream.flush()
    x, y, count = data.batch_at(stream, 0, 2, 8, 11, device=cuda_device)
    assert count == 11 and x.shape == y.shape == (2, 8)
    assert x.is_cuda and x.dtype == y.dtype == torch.int64
    assert int((y != -100).sum()) == 11
    assert y.flatten()[:11].tolist() == list(range(1, 12))
    ex, ey, _ = oracle.batch_at(stream, 0, 2, 8, 11)
    assert np.array_equal(x.cpu().numpy(), ex) and np.array_equal(y.cpu().numpy(), ey)


@pytest.mark.parametrize("resident", [False, True])
def test_batch_at_walks_a_stream_like_the_oracle(cuda_device, resident):
    rng = np.random.default_rng(7)
    stream = rng.integers(0, 65536, 33 * 512 * 3 + 1001).astype(np.uint16)
    stream[:4] = [65535, 0, 50256, 32768]
    source = data.DeviceTokens(stream, cuda_device) if resident else stream
    limit = len(stream) - 1
    cursor = 0
    while True:
        try:
            x, y, count = data.batch_at(source, cursor, 33, 512, limit, device=cuda_device)
        except StopIteration:
            break
        ex, ey, ecount = oracle.batch_at(stream, cursor, 33, 512, limit)
        assert count == ecount
        assert np.array_equal(x.cpu().numpy(), ex) and np.array_equal(y.cpu().numpy(), ey)
        cursor += count
    assert cursor == limit


def test_batch_at_errors(cuda_device):
    stream = np.arange(100, dtype=np.uint16)
    with pytest.raises(StopIteration):
        data.batch_at(stream, 99, 2, 8, 99, device=cuda_device)
    with pytest.raises(ValueError, match="past the end"):
        data.batch_at(stream, 0, 2, 64, 1000, device=cuda_device)
    with pytest.raises(ValueError, match="uint16"):
        data.batch_at(stream.astype(np.int32), 0, 2, 8, 50, device=cuda_device)
    with pytest.raises(ValueError, match="no CPU path"):
        data.batch_at(stream, 0, 2, 8, 50, device="cpu")


def make_ids(kind, batch, seq, vocab, seed):
    g = np.random.default_rng(seed)
    if kind == "uniform":
        ids = g.integers(0, vocab, (batch, seq))
    elif kind == "heavy":
        ids = g.integers(0, vocab, (batch, seq))
        hot = g.random((batch, seq)) < 0.5
        ids[hot] = g.integers(0, 4, int(hot.sum()))
    elif kind == "single":
        ids = np.full((batch, seq), vocab - 1)
    elif kind == "bad":
        ids = g.integers(0, vocab, (batch, seq))
        ids.flat[::7] = vocab
        ids.flat[3::11] = -5
    return ids.astype(np.int64)


CASES = [  # kind, batch, seq, vocab, max_seq, d
    ("uniform", 33, 512, 50257, 1024, 256),
    ("heavy", 16, 2048, 50257, 2048, 1024),
    ("heavy", 3, 37, 101, 64, 36),
    ("single", 5, 100, 7, 128, 1100),
    ("bad", 4, 64, 300, 64, 64),
    ("uniform", 1, 1, 5, 1, 4),
]


@pytest.mark.parametrize("kind,batch,seq,vocab,max_seq,d", CASES)
def test_forward_matches_oracle(cuda_device, kind, batch, seq, vocab, max_seq, d):
    g = torch.Generator().manual_seed(11)
    tok = torch.randn(vocab, d, generator=g)
    pos = torch.randn(max_seq, d, generator=g)
    ids = make_ids(kind, batch, seq, vocab, 1)
    out = embedding.embed(torch.from_numpy(ids).to(cuda_device), tok.to(cuda_device),
                          pos.to(cuda_device))
    ref = oracle.embed_fwd(ids, tok.numpy(), pos.numpy())
    got = out.cpu().numpy()
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(got[~np.isnan(ref)], ref[~np.isnan(ref)])


@pytest.mark.parametrize("accumulate", [False, True])
@pytest.mark.parametrize("kind,batch,seq,vocab,max_seq,d", CASES)
def test_backward_matches_oracle_bitwise(cuda_device, kind, batch, seq, vocab, max_seq, d,
                                         accumulate):
    from reversability_amd._hip import _stream, library
    g = torch.Generator().manual_seed(12)
    ids = make_ids(kind, batch, seq, vocab, 2)
    dout = torch.randn(batch, seq, d, generator=g)
    base_tok = torch.randn(vocab, d, generator=g)
    base_pos = torch.randn(max_seq, d, generator=g)
    ids_d = torch.from_numpy(ids).to(cuda_device)
    dtok = base_tok.to(cuda_device) if accumulate else torch.full((vocab, d), float("nan"), device=cuda_device)
    dpos = base_pos.to(cuda_device) if accumulate else torch.full((max_seq, d), float("nan"), device=cuda_device)
    lib = library()
    nbytes = lib.rv_embed_bwd_workspace_bytes(batch * seq, vocab, d)
    assert nbytes > 0
    ws = torch.empty(nbytes, dtype=torch.uint8, device=cuda_device)
    dout_d = dout.to(cuda_device)
    assert lib.rv_embed_bwd(ids_d.data_ptr(), batch, seq, dout_d.data_ptr(), vocab, max_seq, d,
                            dtok.data_ptr(), int(accumulate), dpos.data_ptr(), int(accumulate),
                            ws.data_ptr(), nbytes, _stream(dout_d)) == 0
    etok, epos = oracle.embed_bwd(ids, dout.numpy(), vocab, max_seq,
                                  dtok=base_tok.numpy().copy() if accumulate else None,
                                  dpos=base_pos.numpy().copy() if accumulate else None)
    assert np.array_equal(dtok.cpu().numpy(), etok)
    assert np.array_equal(dpos.cpu().numpy(), epos)
    # deterministic: a second call gives the same bits
    dtok2 = torch.empty(vocab, d, device=cuda_device)
    assert lib.rv_embed_bwd(ids_d.data_ptr(), batch, seq, dout_d.data_ptr(), vocab, max_seq, d,
                            dtok2.data_ptr(), 0, None, 0, ws.data_ptr(), nbytes,
                            _stream(dout_d)) == 0
    if not accumulate:
        assert torch.equal(dtok2, dtok)


@pytest.mark.parametrize("kind,batch,seq,vocab,max_seq,d", CASES[:4])
def test_autograd_matches_torch_embedding(cuda_device, kind, batch, seq, vocab, max_seq, d):
    g = torch.Generator().manual_seed(13)
    tok = torch.randn(vocab, d, generator=g).to(cuda_device)
    pos = torch.randn(max_seq, d, generator=g).to(cuda_device)
    ids = torch.from_numpy(make_ids(kind, batch, seq, vocab, 3)).to(cuda_device)
    dout = torch.randn(batch, seq, d, generator=g).to(cuda_device)
    t1, p1 = tok.clone().requires_grad_(True), pos.clone().requires_grad_(True)
    out = embedding.embed(ids, t1, p1)
    out.backward(dout)
    t2, p2 = tok.clone().requires_grad_(True), pos.clone().requires_grad_(True)
    ref = torch.nn.functional.embedding(ids, t2) + torch.nn.functional.embedding(
        torch.arange(seq, device=cuda_device), p2)
    ref.backward(dout)
    assert torch.equal(out, ref)
    # fp32 sums in different orders: bound by count * 2^-24 * sum |terms|
    flat = ids.reshape(-1)
    abs_tok = torch.zeros_like(tok).index_add_(0, flat, dout.reshape(-1, d).abs())
    count = torch.bincount(flat, minlength=vocab).float()[:, None]
    assert ((t1.grad - t2.grad).abs() <= count * 2.0 ** -23 * abs_tok + 1e-30).all()
    abs_pos = dout.abs().sum(0)
    assert ((p1.grad[:seq] - p2.grad[:seq]).abs() <= batch * 2.0 ** -23 * abs_pos + 1e-30).all()
    assert (p1.grad[seq:] == 0).all()


def test_into_grad_adds_to_existing_grad(cuda_device):
    g = torch.Generator().manual_seed(14)
    vocab, max_seq, d, batch, seq = 1000, 64, 128, 4, 64
    tok = torch.randn(vocab, d, generator=g).to(cuda_device).requires_grad_(True)
    pos = torch.randn(max_seq, d, generator=g).to(cuda_device).requires_grad_(True)
    ids = torch.from_numpy(make_ids("heavy", batch, seq, vocab, 4)).to(cuda_device)
    dout = torch.randn(batch, seq, d, generator=g).to(cuda_device)
    head = torch.randn(vocab, d, generator=g).to(cuda_device)
    # dense (returned) gradient for reference
    embedding.embed(ids, tok, pos).backward(dout)
    dense = tok.grad.clone()
    tok.grad = head.clone()
    pos.grad = None
    embedding.embed(ids, tok, pos, into_grad=True).backward(dout)
    assert torch.equal(tok.grad, head + dense)
    # with no grad yet the dense gradient is returned
    tok.grad = None
    embedding.embed(ids, tok, pos, into_grad=True).backward(dout)
    assert torch.equal(tok.grad, dense)


def test_embed_rejects_uncovered_inputs(cuda_device):
    tok = torch.randn(10, 6, device=cuda_device)
    pos = torch.randn(8, 6, device=cuda_device)
    ids = torch.zeros(2, 4, dtype=torch.int64, device=cuda_device)
    with pytest.raises(ValueError, match="multiple of 4"):
        embedding.embed(ids, tok, pos)
    with pytest.raises(ValueError):
        embedding.embed(ids.cpu(), tok.cpu()[:, :4].contiguous(), pos.cpu()[:, :4].contiguous())
