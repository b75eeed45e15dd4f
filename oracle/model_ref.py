"""Functional CPU restatement of the decoder and both reversible integrators.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  It shares no code with
``reversability_amd``: parameters come in as a plain ``{name: tensor}`` dict
(state-dict names of src/reversibility/model.py), attention is an explicit
causal softmax (not SDPA), and gradients come from ordinary autograd through
the unrolled recurrence -- what the reference's ``backward_mode='autograd'``
computes (src/reversibility/reversible.py:95-97).

    rms_norm       src/reversibility/model.py:62,64,79 (nn.RMSNorm, eps = finfo.eps)
    attention      src/reversibility/model.py:26-45
    mlp            src/reversibility/model.py:48-56
    midpoint step  src/reversibility/reversible.py:16-25  (p, q) -> (q, p + 2h f(q))
    euler step     src/reversibility/reversible.py:21-25  q' = q + A(p); p' = p + M(q')
    logits         src/reversibility/reversible.py:100-107 (tied head, final norm)
    reconstruction src/reversibility/reversible.py:35-69 (the stack's backward:
                   per layer, reversed, invert the step without a graph,
                   recompute it with one and take its VJP) -- the reference's
                   CPU training path, timed as the step's CPU baseline
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F


def rms_norm(x, w):
    eps = torch.finfo(x.dtype).eps
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


def attention(x, qkv_w, proj_w, n_heads):
    b, t, d = x.shape
    hd = d // n_heads
    qkv = x @ qkv_w.t()
    q, k, v = (qkv[..., i * d:(i + 1) * d].reshape(b, t, n_heads, hd).transpose(1, 2)
               for i in range(3))
    scores = (q @ k.transpose(-1, -2)) / math.sqrt(hd)
    mask = torch.ones(t, t, dtype=torch.bool).triu(1)
    scores = scores.masked_fill(mask, float("-inf"))
    y = torch.softmax(scores, -1) @ v
    return y.transpose(1, 2).reshape(b, t, d) @ proj_w.t()


def mlp(x, up_w, down_w):
    u = x @ up_w.t()
    f = u.shape[-1] // 2
    g, v = u[..., :f], u[..., f:]
    return (g * torch.sigmoid(g) * v) @ down_w.t()


def _A(params, i, x, n_heads):
    pre = f"blocks.{i}."
    return attention(rms_norm(x, params[pre + "attn_norm.weight"]), params[pre + "attn.qkv.weight"],
                     params[pre + "attn.proj.weight"], n_heads)


def _M(params, i, x):
    pre = f"blocks.{i}."
    return mlp(rms_norm(x, params[pre + "mlp_norm.weight"]), params[pre + "mlp.up.weight"],
               params[pre + "mlp.down.weight"])


def core(params, x, n_layers, n_heads, method, h=0.5, record=None):
    """The integrator stack from p = q = x; returns the head input state."""
    p = q = x
    if record is not None:
        record.append((p, q))
    for i in range(n_layers):
        if method == "midpoint":
            a = _A(params, i, q, n_heads)
            force = a + _M(params, i, q + a)
            p, q = q, p + 2 * h * force
        elif method == "euler":
            q = q + _A(params, i, p, n_heads)
            p = p + _M(params, i, q)
        else:  # plain residual blocks (BaselineLM)
            x = q + _A(params, i, q, n_heads)
            p = q = x + _M(params, i, x)
        if record is not None:
            record.append((p, q))
    return q if method in ("midpoint", "baseline") else p


def logits(params, ids, n_layers, n_heads, method, h=0.5):
    t = ids.shape[1]
    x = params["token_embedding.weight"][ids] + params["position_embedding.weight"][:t]
    hidden = core(params, x, n_layers, n_heads, method, h)
    return rms_norm(hidden, params["final_norm.weight"]) @ params["token_embedding.weight"].t()


def loss_and_grads(state, ids, labels, n_layers, n_heads, method, h=0.5, dtype=torch.float32,
                   reduction="mean"):
    """Cross-entropy and its gradients for every parameter of ``state``.

    ``state`` is a state dict (the tied ``lm_head.weight`` is dropped; the head
    uses the token embedding).  Returns (loss, {name: grad}) on the CPU.
    """
    params = {k: v.detach().to("cpu", dtype).clone().requires_grad_(True)
              for k, v in state.items() if k != "lm_head.weight"}
    out = logits(params, ids.cpu(), n_layers, n_heads, method, h)
    loss = F.cross_entropy(out.flatten(0, 1), labels.cpu().flatten(), ignore_index=-100,
                           reduction=reduction)
    loss.backward()
    return loss.detach(), {k: v.grad for k, v in params.items()}


def _step(params, i, p, q, n_heads, method, h):
    if method == "midpoint":
        a = _A(params, i, q, n_heads)
        return q, p + 2 * h * (a + _M(params, i, q + a))
    q = q + _A(params, i, p, n_heads)
    return p + _M(params, i, q), q


def _inverse(params, i, p, q, n_heads, method, h):
    if method == "midpoint":
        a = _A(params, i, p, n_heads)
        return q - 2 * h * (a + _M(params, i, p + a)), p
    p0 = p - _M(params, i, q)
    return p0, q - _A(params, i, p0, n_heads)


def loss_and_grads_reconstruct(state, ids, labels, n_layers, n_heads, method, h=0.5,
                               dtype=torch.float32, reduction="mean"):
    """``loss_and_grads`` through the reconstruction backward: the stack runs
    without a graph, the head and loss are differentiated at its final pair,
    then each layer, last first, is inverted (no graph), recomputed with a
    graph and differentiated with the pair's incoming gradients
    (src/reversibility/reversible.py:35-69).  Midpoint and Euler only."""
    if method not in ("midpoint", "euler"):
        raise ValueError("reconstruction needs a reversible method")
    params = {k: v.detach().to("cpu", dtype).clone().requires_grad_(True)
              for k, v in state.items() if k != "lm_head.weight"}
    ids, labels = ids.cpu(), labels.cpu()
    t = ids.shape[1]
    emb = params["token_embedding.weight"][ids] + params["position_embedding.weight"][:t]
    with torch.no_grad():
        p = q = emb.detach()
        for i in range(n_layers):
            p, q = _step(params, i, p, q, n_heads, method, h)
    p, q = p.requires_grad_(True), q.requires_grad_(True)
    head_in = q if method == "midpoint" else p
    out = rms_norm(head_in, params["final_norm.weight"]) @ params["token_embedding.weight"].t()
    loss = F.cross_entropy(out.flatten(0, 1), labels.flatten(), ignore_index=-100,
                           reduction=reduction)
    loss.backward()
    dp = p.grad if p.grad is not None else torch.zeros_like(p)
    dq = q.grad if q.grad is not None else torch.zeros_like(q)
    p, q = p.detach(), q.detach()
    for i in reversed(range(n_layers)):
        with torch.no_grad():
            p0, q0 = _inverse(params, i, p, q, n_heads, method, h)
        p0, q0 = p0.requires_grad_(True), q0.requires_grad_(True)
        np_, nq = _step(params, i, p0, q0, n_heads, method, h)
        torch.autograd.backward((np_, nq), (dp, dq))
        dp, dq = p0.grad, q0.grad
        p, q = p0.detach(), q0.detach()
    emb.backward(dp + dq)  # the boundary p = q = embedding
    return loss.detach(), {k: v.grad for k, v in params.items()}
