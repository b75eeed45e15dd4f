"""Per-layer workspace reduction: token-tiled MLP and split midpoint backward.

Restates src/reversibility/optimized_v3.py:10-192.

``TiledMLP`` saves only the normalized input and the two weights and
recomputes bounded token tiles in backward.  Its backward is written out
(instead of rebuilding an autograd graph per tile and calling
``autograd.grad``): per tile it recomputes ``u = x W_up^T`` and ``o = swiglu(u)``
-- the down projection output is not needed for gradients and is not
recomputed -- then

    d_o    = dy W_down          dW_down += fp32(dy^T o)
    du     = swiglu_bwd(u, d_o)
    dx     = fp32(du W_up)      dW_up   += fp32(du^T x)

with the same casts autocast's ``F.linear`` applies (inputs and weights to the
autocast dtype; gradients of fp32 leaves cast back to fp32) and the same
per-tile fp32 accumulation order as the reference's ``add_``.
"""
from __future__ import annotations

import types

import torch
import torch.nn.functional as F
from torch.autograd.function import once_differentiable

from . import paths as _paths
from .kernels_v3 import add_rms_norm, add_rms_norm_pass, midpoint_rms_norm, rms_norm_pass
from .optimized import ReusedMidpoint, amp_context, hidden_states
from .residual import eager_active, eager_updates, midpoint_step


def mlp_value(x, up, down, fused):
    """down(swiglu(x up^T)) under the caller's autocast (optimized_v3.py:10-18)."""
    u = F.linear(x, up)
    if fused:
        from .kernels import FusedSwiGLU
        value = FusedSwiGLU.apply(u)
    else:
        gate, value = u.chunk(2, -1)
        value = F.silu(gate) * value
    return F.linear(value, down)


def _swiglu_forward(u, fused):
    if fused:
        from .kernels import _validate
        from ._hip import ops
        _validate(u)
        return ops.swiglu_fwd(u)
    gate, value = u.chunk(2, -1)
    return F.silu(gate) * value


def _swiglu_backward(u, d_o, fused):
    if fused:
        from ._hip import ops
        return ops.swiglu_bwd(u, d_o.contiguous())
    with torch.enable_grad():
        leaf = u.detach().requires_grad_(True)
        gate, value = leaf.chunk(2, -1)
        out = F.silu(gate) * value
        du, = torch.autograd.grad(out, leaf, d_o)
    return du


def tile_forward(x, up_c, down_c, fused, compute_dtype, need_output=True):
    """One tile of the MLP in ``compute_dtype`` (weights already cast):
    returns (x_c, u, o, y)."""
    x_c = x.to(compute_dtype)
    u = torch.mm(x_c, up_c.t())
    o = _swiglu_forward(u, fused)
    y = torch.mm(o, down_c.t()) if need_output else None
    return x_c, u, o, y


def _compute_dtype(x, amp, amp_dtype):
    if amp and x.dtype == torch.float32:
        return amp_dtype
    return x.dtype


def _use_mfma(x, up, down, fused, cdt):
    """The fused MFMA path covers fp16 compute with fp32 weights at widths that
    are multiples of 128; other cases keep torch's GEMMs (and the fused SwiGLU
    kernel when ``fused``)."""
    from . import mlp
    return fused and cdt == torch.float16 and mlp.supported(x, up, down)


def _record_mlp_path(x, up, down, fused, cdt, mfma):
    if mfma:
        _paths.took("tiled_mlp", "mfma")
    elif fused and x.is_cuda:
        _paths.took("tiled_mlp", "torch-gemm",
                    f"MFMA MLP needs fp16 compute and widths that are multiples of 128 "
                    f"(d={x.shape[-1]}, f={down.shape[1]}, compute {cdt})")
    else:  # the unfused computation the caller asked for, or a CPU tensor
        _paths.took("tiled_mlp", "torch-gemm")


class TiledMLP(torch.autograd.Function):
    """Save only the normalized input and weights; recompute token tiles in backward.

    Attention still sees all sequences; each optimizer update consumes one whole
    physical batch.  Parameter gradients return through autograd inputs.

    On ROCm tensors under fp16 autocast with ``fused`` the tile's GEMMs are the
    MFMA kernels of ``reversability_amd.mlp`` with SwiGLU (and its backward)
    fused into the GEMM epilogues.
    """

    @staticmethod
    def forward(ctx, x, up, down, tokens, fused, keep_tiles=False, need_output=True):
        if tokens < 1:
            raise ValueError("Positive MLP tile size required")
        ctx.tokens, ctx.fused = tokens, fused
        ctx.tiles = None
        ctx.device = x.device.type
        ctx.amp = torch.is_autocast_enabled(ctx.device)
        ctx.dtype = torch.get_autocast_dtype(ctx.device)
        cdt = _compute_dtype(x, ctx.amp, ctx.dtype)
        flat = x.reshape(-1, x.shape[-1])
        output = torch.empty((flat.shape[0], down.shape[0]), device=x.device, dtype=cdt)
        mfma = _use_mfma(flat, up, down, fused, cdt)
        _record_mlp_path(flat, up, down, fused, cdt, mfma)
        if not need_output and not (keep_tiles and mfma):
            # the output is only differentiated and there are no tiles to keep:
            # nothing to compute (the backward recomputes its tiles)
            ctx.save_for_backward(x, up, down)
            return output.reshape(*x.shape[:-1], down.shape[0])
        if mfma:
            from . import mlp
            # autocast's casts, once per call: the same fp16 values F.linear
            # would produce on every tile
            x16 = mlp.cast_f16(flat.contiguous())
            up16, down16 = mlp.cast_weight(up), mlp.cast_weight(down)
            tiles = [] if keep_tiles else None
            for start in range(0, flat.shape[0], tokens):
                o, u = mlp.up_swiglu(x16[start:start + tokens], up16, keep_u=keep_tiles)
                if need_output:
                    mlp.down(o, down16, output[start:start + tokens])
                if keep_tiles:
                    tiles.append((o, u))
            ctx.tiles = tiles
            del x16, up16, down16
            ctx.save_for_backward(x, up, down)
            return output.reshape(*x.shape[:-1], down.shape[0])
        with torch.autocast(ctx.device, enabled=False):
            # autocast's F.linear casts the weights on every call; one cast per
            # call here gives the same values
            up_c, down_c = up.to(cdt), down.to(cdt)
            for start in range(0, flat.shape[0], tokens):
                *_, y = tile_forward(flat[start:start + tokens], up_c, down_c, fused, cdt,
                                     need_output=need_output)
                if need_output:
                    output[start:start + tokens].copy_(y)
        ctx.save_for_backward(x, up, down)
        return output.reshape(*x.shape[:-1], down.shape[0])

    @staticmethod
    @once_differentiable
    def backward(ctx, gradient):
        x, up, down = ctx.saved_tensors
        cdt = _compute_dtype(x, ctx.amp, ctx.dtype)
        flat = x.reshape(-1, x.shape[-1])
        dy = gradient.reshape(-1, gradient.shape[-1]).to(cdt)
        dx = torch.empty_like(flat)
        if _use_mfma(flat, up, down, ctx.fused, cdt):
            from . import mlp
            x16, dy = mlp.cast_f16(flat.contiguous()), dy.contiguous()
            up16, down16 = mlp.cast_weight(up), mlp.cast_weight(down)
            dup, ddown = torch.empty_like(up), torch.empty_like(down)
            tiles, ctx.tiles = ctx.tiles, None
            for i, start in enumerate(range(0, flat.shape[0], ctx.tokens)):
                stop = start + ctx.tokens
                x_t, g = x16[start:stop], dy[start:stop]
                if tiles is not None:  # kept by the forward: the same values
                    o, u = tiles[i]
                    tiles[i] = None
                else:
                    o, u = mlp.up_swiglu(x_t, up16, keep_u=True)
                du = mlp.dgate(g, down16, u)
                mlp.dx(du, up16, dx[start:stop])
                mlp.wgrad(g, o, du, x_t, ddown, dup, accumulate=i > 0)
                del o, u, du
            return dx.reshape_as(x), dup, ddown, None, None, None, None
        dup = ddown = None
        with torch.autocast(ctx.device, enabled=False):
            up_c, down_c = up.to(cdt), down.to(cdt)
            for start in range(0, flat.shape[0], ctx.tokens):
                stop = start + ctx.tokens
                x_c, u, o, _ = tile_forward(flat[start:stop], up_c, down_c, ctx.fused, cdt,
                                            need_output=False)
                g = dy[start:stop]
                d_o = torch.mm(g, down_c)
                tile_ddown = torch.mm(g.t(), o).to(down.dtype)
                du = _swiglu_backward(u, d_o, ctx.fused)
                dx[start:stop].copy_(torch.mm(du, up_c))
                tile_dup = torch.mm(du.t(), x_c).to(up.dtype)
                # first tile initialises the fp32 accumulators (0 + t == t)
                ddown = tile_ddown if ddown is None else ddown.add_(tile_ddown)
                dup = tile_dup if dup is None else dup.add_(tile_dup)
                del x_c, u, o, g, d_o, du, tile_ddown, tile_dup
        if dup is None:  # no rows
            dup, ddown = torch.zeros_like(up), torch.zeros_like(down)
        return dx.reshape_as(x), dup, ddown, None, None, None, None


# The model's switches for SplitMidpoint (paths.ReconstructionPaths):
#   keep_split_attention  the backward evaluates each layer's attention twice on
#       the same input -- under no_grad for the inversion, then with gradients
#       for its VJP; with the switch on, the first evaluation is made with
#       gradients and its graph (one layer's attention, held through the MLP
#       VJP) serves the VJP: the same values, one attention evaluation less;
#   fuse_midpoint_norm    each midpoint update made together with the attention
#       norm of the layer that reads it next (forward and reconstruction).


class SplitMidpoint(torch.autograd.Function):
    """MLP VJP first, then the attention VJP (optimized_v3.py:66-117).

    A detached attention proxy carries the force's dependence on attention, so
    the MLP graph can be released before the attention VJP.  The reference
    recomputes attention for that VJP (its disclosed extra-compute trade-off);
    with the model's ``keep_split_attention`` the inversion's attention graph
    is kept instead.
    """

    @staticmethod
    def forward(ctx, p, q, blocks, h, *parameters):
        ctx.blocks, ctx.h = blocks, h
        ctx.eager = eager_active()
        ctx.device = p.device.type
        ctx.amp = torch.is_autocast_enabled(ctx.device)
        ctx.dtype = torch.get_autocast_dtype(ctx.device)
        from .reversible import midpoint_terms
        fuse_norm = _paths.of(blocks).fuse_midpoint_norm
        normed = None  # the next block's attn_norm(q), made with the midpoint update
        for i, block in enumerate(blocks):
            if normed is None:
                attention, mlp = midpoint_terms(block, q)
            else:
                attention = block.attn(normed)
                mlp = block.mlp(add_rms_norm(q, attention, block.mlp_norm)[1])
            lower = blocks[i + 1] if i + 1 < len(blocks) else None
            if fuse_norm and lower is not None:
                nxt, pre = midpoint_rms_norm(p, attention, mlp, 2 * h, +1, lower.attn_norm)
                normed = pre[0] if pre is not None else None
            else:
                nxt, normed = midpoint_step(p, attention, mlp, 2 * h, +1), None
            p, q = q, nxt
            del attention, mlp
        ctx.save_for_backward(p, q, *parameters)
        return p, q

    @staticmethod
    @once_differentiable
    def backward(ctx, dp, dq):
        p, q, *_ = ctx.saved_tensors
        grads: list = []
        scale = 2 * ctx.h
        settings = _paths.of(ctx.blocks)
        keep_attention = settings.keep_split_attention
        fuse_norm = settings.fuse_midpoint_norm and keep_attention
        # No autocast weight-cast cache: the no_grad attention pass below would
        # otherwise leave history-free fp16 weight casts for the grad-enabled
        # rebuild (torch <= 2.10); casts are deterministic, values unchanged.
        with torch.autocast(ctx.device, enabled=ctx.amp, dtype=ctx.dtype,
                            cache_enabled=False), eager_updates(ctx.eager):
            pre_p = None  # attn_norm(p) of this block, made with the previous inversion
            for index in reversed(range(len(ctx.blocks))):
                block = ctx.blocks[index]
                lower = ctx.blocks[index - 1] if index > 0 else None
                if keep_attention:  # its graph serves the attention VJP below
                    with torch.enable_grad():
                        attn_input = p.detach().requires_grad_(True)
                        attn_pass, normed = rms_norm_pass(attn_input, block.attn_norm, pre_p)
                        attention = block.attn(normed)
                else:
                    with torch.no_grad():
                        attention = block.attn(block.attn_norm(p))
                with torch.enable_grad():
                    previous_q = p.detach().requires_grad_(True)
                    proxy = attention.detach().requires_grad_(True)
                    # previous_q is also an output of this step: its two
                    # gradients are summed in the norm's backward pass
                    q_pass, mlp_in = add_rms_norm_pass(previous_q, proxy, block.mlp_norm)
                    mlp = block.mlp(mlp_in)
                    if fuse_norm and lower is not None:
                        # previous_p with the lower block's attn_norm of it
                        previous_p, pre_p = midpoint_rms_norm(q, proxy.detach(), mlp.detach(),
                                                              scale, -1, lower.attn_norm)
                    else:
                        with torch.no_grad():
                            previous_p = midpoint_step(q, proxy.detach(), mlp.detach(), scale,
                                                       -1)
                        pre_p = None
                    previous_p.requires_grad_(True)
                    # only differentiated: its value is never read
                    next_q = midpoint_step(previous_p, proxy, mlp, scale, +1, graph_only=True)
                    mlp_parameters = (*block.mlp_norm.parameters(), *block.mlp.parameters())
                    local = torch.autograd.grad((q_pass, next_q),
                                                (previous_p, previous_q, proxy, *mlp_parameters),
                                                (dp, dq))
                next_dp, q_mlp, attention_cotangent = local[:3]
                mlp_grads = local[3:]
                del proxy, mlp, next_q, local, q_pass, mlp_in
                with torch.enable_grad():
                    if not keep_attention:
                        attn_input = previous_q.detach().requires_grad_(True)
                        attn_pass, normed = rms_norm_pass(attn_input, block.attn_norm)
                        attention = block.attn(normed)
                    attention_parameters = (*block.attn_norm.parameters(), *block.attn.parameters())
                    # q's two gradients (MLP graph, attention graph) are summed in
                    # the attention norm's backward pass: q_mlp enters as the
                    # gradient of the norm's pass-through output
                    attn_local = torch.autograd.grad((attention, attn_pass),
                                                     (attn_input, *attention_parameters),
                                                     (attention_cotangent, q_mlp))
                dp, dq = next_dp, attn_local[0]
                by_id = {id(w): g for w, g in zip((*attention_parameters, *mlp_parameters),
                                                  (*attn_local[1:], *mlp_grads))}
                grads[0:0] = [by_id[id(w)] for w in block.parameters()]
                p, q = previous_p.detach(), previous_q.detach()
                del attn_input, attn_pass, normed, attention, attn_local, attention_cotangent, q_mlp, by_id, mlp_grads
        return (dp, dq, None, None, *grads)


def _fused_head(hidden, weight, labels, denominator, chunk_tokens, scaler, precision, device):
    """The chunk loop of cached_head_backward for the fused fp16 loss, without
    building an autograd graph for the head: per chunk the fp16 logits (padded
    row stride), the fused cross-entropy forward and backward with the upstream
    gradient d(scale * loss / denominator)/d loss = scale / denominator, and
    the two gradient GEMMs (kernels.tied_head_ce).  Same values as the autograd
    loop: the head's fp16 gradient of each chunk is widened and added to the
    tied weight's gradient, the hidden-state gradient of each chunk fills its
    rows, and one core backward follows."""
    from .kernels import padded_head, tied_head_ce
    flat = hidden.detach().reshape(-1, hidden.shape[-1])
    x16 = flat if flat.dtype == torch.float16 else flat.to(torch.float16)
    x16 = x16.contiguous()
    head16 = padded_head(weight.detach())
    vocab = weight.shape[0]
    one = torch.ones((), device=device, dtype=torch.float32)
    grad = (one if scaler is None else scaler.scale(one)) / denominator
    targets = labels.reshape(-1)
    dflat = torch.empty_like(flat)
    total = torch.zeros((), device=device, dtype=torch.float32)
    for start in range(0, targets.numel(), chunk_tokens):
        stop = start + chunk_tokens
        rows = dflat[start:stop]
        direct = rows.dtype == torch.float16 and rows.is_contiguous()
        loss, dx16, dw16 = tied_head_ce(x16[start:stop], head16, vocab, targets[start:stop],
                                        grad.reshape(1), dx_out=rows if direct else None)
        if not direct:
            rows.copy_(dx16)
        chunk_grad = dw16.to(weight.dtype)
        if weight.grad is None:
            weight.grad = chunk_grad
        else:
            weight.grad.add_(chunk_grad)
        total += loss.detach().float()
        del dx16, dw16, chunk_grad
    del head16, x16
    with amp_context(device, precision):
        hidden.backward(dflat.reshape_as(hidden))
    return total


def install_v3(model, *, core_mode="reference", mlp_tokens=0, swiglu=False, rmsnorm=False,
               keep_mlp_tiles=False, paths=None):
    """Wire the optimized core, tiled MLP, fused SwiGLU and fused RMSNorm
    (optimized_v3.py:120-148).  Idempotent for one configuration; raises on a
    conflicting reinstall, a non-midpoint optimized core, or a biased MLP.

    ``paths`` (not in the reference): the model's reconstruction switches
    (``paths.ReconstructionPaths``; default all on), recorded on the model.

    ``keep_mlp_tiles`` (not in the reference): a TiledMLP forward that runs with
    gradients enabled keeps its tiles' SwiGLU input and output for its backward
    instead of recomputing them there.  In the reconstruction backward that is
    one layer's tiles at a time (C5: 0.8 GB), and one up-projection GEMM per
    layer and step less; the kept values are the ones the recompute would
    produce, bit for bit."""
    settings = paths if paths is not None else _paths.DEFAULT
    signature = (core_mode, mlp_tokens, swiglu, rmsnorm, keep_mlp_tiles, settings)
    if hasattr(model, "_v3_signature"):
        if model._v3_signature != signature:
            raise ValueError("Cannot replace an installed v3 configuration")
        return model
    _paths.configure(model, settings)
    if core_mode != "reference":
        if getattr(model, "method", None) != "midpoint" or model.backward_mode != "reconstruct":
            raise ValueError("Optimized core requires reconstructed midpoint")
        core_function = {"reuse": ReusedMidpoint, "split": SplitMidpoint}[core_mode]

        def core(self, x):
            _, y = core_function.apply(x, x, self.blocks, self.step_size, *self.blocks.parameters())
            return y
        model.core = types.MethodType(core, model)
    if mlp_tokens:
        for block in model.blocks:
            if block.mlp.up.bias is not None or block.mlp.down.bias is not None:
                raise ValueError("Tiled MLP experiment supports frozen bias=False only")

            def forward(self, x):
                from . import mlp
                return TiledMLP.apply(x, self.up.weight, self.down.weight, mlp_tokens, swiglu,
                                      keep_mlp_tiles and torch.is_grad_enabled(),
                                      mlp.output_wanted(x))
            block.mlp.forward = types.MethodType(forward, block.mlp)
    elif swiglu:
        from .kernels import enable_swiglu
        enable_swiglu(model)
    if rmsnorm:
        from .kernels_v3 import enable_rmsnorm
        # every norm here feeds only fp16-autocast GEMMs (qkv, the MLP's up
        # projection, the tied head), so under fp16 autocast it hands them the
        # fp16 operand directly
        enable_rmsnorm(model, fp16_out=True)
    model._v3_signature = signature
    return model


def cached_head_backward(model, ids, labels, denominator, chunk_tokens, scaler=None,
                         precision="fp32", reuse=False, loss_backend="torch"):
    """Chunked tied-head loss with one head-weight cast per update
    (optimized_v3.py:151-192).  Each chunk's head gradient is promoted to the
    weight dtype before it is added to the tied ``.grad``."""
    if reuse or chunk_tokens < 1 or denominator < 1:
        raise ValueError("Use installed core mode and positive normalization/chunk")
    from . import mlp
    with mlp.weight_cast_cache():  # weights are constant until the optimizer step
        if precision == "fp16" and ids.device.type == "cuda":
            mlp.prefetch_casts(castable_weights(model))
        return _cached_head_backward(model, ids, labels, denominator, chunk_tokens, scaler,
                                     precision, loss_backend)


def castable_weights(model) -> list:
    """The fp32 weights the step's MFMA GEMMs cast to fp16 through
    ``mlp.cast_weight``: the tiled MLP's up and down projections when
    ``install_v3`` tiled the MLP, the attention projections routed through
    ``linear.enable_linear``.  One ``mlp.prefetch_casts`` launch makes all of
    them at the start of a step."""
    tiled = bool(getattr(model, "_v3_signature", (None, 0))[1])
    weights = []
    for block in model.blocks:
        for layer in (block.attn.qkv, block.attn.proj):
            if getattr(layer, "_rv_linear", False):
                weights.append(layer.weight)
        if tiled:
            weights += [block.mlp.up.weight, block.mlp.down.weight]
    return weights


def _cached_head_backward(model, ids, labels, denominator, chunk_tokens, scaler, precision,
                          loss_backend):
    with amp_context(ids.device, precision):
        hidden = hidden_states(model, ids)
    weight = model.lm_head.weight
    if (loss_backend in ("triton", "hip") and precision == "fp16" and ids.device.type == "cuda"
            and weight.dtype == torch.float32):
        _paths.took("tied_head", "fused-ce+hipblaslt")
        return _fused_head(hidden, weight, labels, denominator, chunk_tokens, scaler, precision,
                           ids.device)
    if loss_backend in ("triton", "hip") and ids.device.type == "cuda":
        _paths.took("tied_head", "autograd-chunks",
                    f"the fused head needs fp16 precision and an fp32 weight (got {precision}, "
                    f"{weight.dtype})")
    else:
        _paths.took("tied_head", "autograd-chunks")
    leaf = hidden.detach().reshape(-1, hidden.shape[-1]).requires_grad_(True)
    if ids.device.type != "cuda" or precision == "fp32":
        dtype = weight.dtype
    else:
        dtype = {"fp16": torch.float16, "bf16": torch.bfloat16}[precision]
    head = weight.detach().to(dtype).requires_grad_(True)
    targets = labels.reshape(-1)
    total = torch.zeros((), device=ids.device, dtype=torch.float32)
    from .optimized import _chunk_loss
    for start in range(0, targets.numel(), chunk_tokens):
        with amp_context(ids.device, precision, cache=False):
            logits = F.linear(leaf[start:start + chunk_tokens], head)
            loss = _chunk_loss(logits, targets[start:start + chunk_tokens], loss_backend)
            normalized = loss / denominator
            (normalized if scaler is None else scaler.scale(normalized)).backward()
        chunk_grad = head.grad.detach().to(weight.dtype)
        if weight.grad is None:
            weight.grad = chunk_grad
        else:
            weight.grad.add_(chunk_grad)
        head.grad = None
        total += loss.detach().float()
        del logits, loss, normalized, chunk_grad
    del head
    with amp_context(ids.device, precision):
        hidden.backward(leaf.grad.reshape_as(hidden))
    return total
