"""Token pipeline: the uint16 token file to one micro-batch of int64 inputs
and targets on the device (scripts/train_baseline.py:50-63, ``batch_at``).

The reference slices a ``np.memmap`` of uint16 tokens, widens the window to
int64 on the host, pads it to whole sequences (inputs with 0, targets with
-100) and the trainer copies both int64 tensors to the GPU: 16 bytes per token
over PCIe.  Here only the uint16 window travels (2 bytes per token; nothing at
all once the stream is resident in HBM, see :class:`DeviceTokens`) and the
widening, shifting and padding run on the GPU (``rv_batch_from_tokens``).

``batch_at`` keeps the reference's signature, target accounting and error
behaviour (``StopIteration`` once ``cursor`` reaches ``target_limit``) and
returns device tensors.
"""
from __future__ import annotations

import numpy as np
import torch

from ._hip import _check, _stream, library

IGNORE_INDEX = -100


def _require_cuda(device) -> torch.device:
    device = torch.device(device)
    if device.type != "cuda":
        raise ValueError("batch_at builds batches on the ROCm device; no CPU path")
    return device


class DeviceTokens:
    """A uint16 token stream held in HBM (2 bytes per token: a 10B-token
    corpus is 20 GB of a 288 GB device), uploaded once in pieces of
    ``chunk_tokens`` so no host copy of the whole file is made."""

    def __init__(self, data, device="cuda", chunk_tokens: int = 1 << 26):
        device = _require_cuda(device)
        array = np.asarray(data)
        if array.ndim != 1 or array.dtype != np.uint16:
            raise ValueError("DeviceTokens expects a 1-D uint16 token stream")
        self.tokens = torch.empty(array.shape[0], dtype=torch.int16, device=device)
        for start in range(0, array.shape[0], chunk_tokens):
            piece = np.ascontiguousarray(array[start:start + chunk_tokens]).view(np.int16)
            self.tokens[start:start + piece.shape[0]].copy_(torch.from_numpy(piece))

    @property
    def device(self) -> torch.device:
        return self.tokens.device

    def __len__(self) -> int:
        return self.tokens.shape[0]


def batch_at(data, cursor: int, batch_size: int, sequence_length: int, target_limit: int,
             device=None):
    """(x, y, count): x, y int64 [ceil(count / sequence_length), sequence_length]
    on the device, count = min(batch_size * sequence_length, target_limit - cursor)
    real targets (scripts/train_baseline.py:50-63).

    ``data`` is a host uint16 array / ``np.memmap`` (then ``device`` names the
    GPU) or a :class:`DeviceTokens`."""
    count = min(batch_size * sequence_length, target_limit - cursor)
    if count <= 0:
        raise StopIteration
    if cursor < 0 or sequence_length <= 0:
        raise ValueError("cursor must be >= 0 and sequence_length > 0")
    if cursor + count + 1 > len(data):
        raise ValueError("token window runs past the end of the stream")
    if isinstance(data, DeviceTokens):
        device = data.device
        window = data.tokens[cursor:cursor + count + 1]
    else:
        device = _require_cuda("cuda" if device is None else device)
        array = np.asarray(data)
        if array.dtype != np.uint16:
            raise ValueError("batch_at expects a uint16 token stream")
        host = torch.from_numpy(np.ascontiguousarray(array[cursor:cursor + count + 1]).view(np.int16))
        window = host.to(device)
    sequences = -(-count // sequence_length)
    x = torch.empty(sequences, sequence_length, dtype=torch.int64, device=device)
    y = torch.empty_like(x)
    _check(library().rv_batch_from_tokens(window.data_ptr(), count, sequence_length, x.data_ptr(),
                                          y.data_ptr(), _stream(x)), "rv_batch_from_tokens")
    return x, y, count
