"""Independent float64 model of one TransformerLM training step, built from torch library
routines (F.embedding, F.rms_norm, F.linear, scaled_dot_product_attention, F.silu,
F.cross_entropy, clip_grad_norm_, torch.optim.AdamW) and torch autograd.

Used only by the tests, to pin the C oracle: a dropped term, a wrong sign or a transposed
operand in the oracle's hand-written backward shows up as a gradient mismatch here.
RoPE has no library routine; its tables are built in numpy float32 from the formula of
include/nn/rope.hpp:122-144 and its math is pinned separately by invariants.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F


def layout(vocab, d, n_layers, f, tied, n_experts=0):
    """(name, shape) in the flat order the oracle and the product arena share."""
    out = [("tok_embeddings.weight", (vocab, d))]
    for l in range(n_layers):
        p = f"layers.{l}."
        out += [(p + "attn.q_proj.weight", (d, d)), (p + "attn.k_proj.weight", (d, d)),
                (p + "attn.v_proj.weight", (d, d)), (p + "attn.out_proj.weight", (d, d))]
        if n_experts:
            out.append((p + "moe.router.gate.weight", (n_experts, d)))
            for e in range(n_experts):
                q = p + f"moe.experts.{e}."
                out += [(q + "gate_proj.weight", (f, d)), (q + "up_proj.weight", (f, d)),
                        (q + "down_proj.weight", (d, f))]
        else:
            out += [(p + "ffn.gate_proj.weight", (f, d)), (p + "ffn.up_proj.weight", (f, d)),
                    (p + "ffn.down_proj.weight", (d, f))]
        out += [(p + "norm1.weight", (d,)), (p + "norm2.weight", (d,))]
    out.append(("norm.weight", (d,)))
    if not tied:
        out.append(("lm_head.weight", (vocab, d)))
    return out


def rope_tables_np(S, hd, base=10000.0):
    half = hd // 2
    i = np.arange(half, dtype=np.float32)
    exponent = (np.float32(2.0) * i) / np.float32(hd)
    freqs = np.float32(1.0) / np.power(np.float32(base), exponent, dtype=np.float32)
    pos = np.arange(S, dtype=np.float32)[:, None]
    ang = (pos * freqs[None, :]).astype(np.float32)
    return np.cos(ang.astype(np.float64)).astype(np.float32), np.sin(ang.astype(np.float64)).astype(np.float32)


def rope(x, cos, sin):
    """x [B, H, S, hd]; half-split rotation."""
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    return torch.cat([x1 * cos - x2 * sin, x1 * sin + x2 * cos], dim=-1)


def lm_step(vocab, d, n_layers, n_heads, f, tied, params_flat, ids, targets, B, S, eps=1e-6, lr=3e-4,
            betas=(0.9, 0.95), adam_eps=1e-8, weight_decay=0.1, max_grad_norm=1.0, dtype=torch.float64,
            n_experts=0, top_k=2, aux_coef=0.01):
    """Returns loss (cross-entropy + the MoE aux losses), pre-clip grad norm, grads, updated params."""
    lay = layout(vocab, d, n_layers, f, tied, n_experts)
    P = {}
    off = 0
    for name, shape in lay:
        n = int(np.prod(shape))
        P[name] = torch.tensor(params_flat[off:off + n].reshape(shape), dtype=dtype, requires_grad=True)
        off += n
    assert off == params_flat.size
    hd = d // n_heads
    cos_np, sin_np = rope_tables_np(S, hd)
    cos = torch.tensor(cos_np, dtype=dtype)[None, None]
    sin = torch.tensor(sin_np, dtype=dtype)[None, None]
    ids_t = torch.tensor(np.asarray(ids).reshape(B, S), dtype=torch.long)
    tgt_t = torch.tensor(np.asarray(targets).reshape(B * S), dtype=torch.long)

    x = F.embedding(ids_t, P["tok_embeddings.weight"])
    aux_total = None
    for l in range(n_layers):
        p = f"layers.{l}."
        h = F.rms_norm(x, (d,), P[p + "norm1.weight"], eps)
        q = F.linear(h, P[p + "attn.q_proj.weight"]).view(B, S, n_heads, hd).transpose(1, 2)
        k = F.linear(h, P[p + "attn.k_proj.weight"]).view(B, S, n_heads, hd).transpose(1, 2)
        v = F.linear(h, P[p + "attn.v_proj.weight"]).view(B, S, n_heads, hd).transpose(1, 2)
        q, k = rope(q, cos, sin), rope(k, cos, sin)
        o = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        o = o.transpose(1, 2).reshape(B, S, d)
        x = x + F.linear(o, P[p + "attn.out_proj.weight"])
        h = F.rms_norm(x, (d,), P[p + "norm2.weight"], eps)
        if n_experts:
            ex = [(P[p + f"moe.experts.{e}.gate_proj.weight"], P[p + f"moe.experts.{e}.up_proj.weight"],
                   P[p + f"moe.experts.{e}.down_proj.weight"]) for e in range(n_experts)]
            y, aux = moe_layer(h.reshape(B * S, d), P[p + "moe.router.gate.weight"], ex, top_k, aux_coef)
            x = x + y.reshape(B, S, d)
            aux_total = aux if aux_total is None else aux_total + aux
        else:
            a = F.silu(F.linear(h, P[p + "ffn.gate_proj.weight"])) * F.linear(h, P[p + "ffn.up_proj.weight"])
            x = x + F.linear(a, P[p + "ffn.down_proj.weight"])
    x = F.rms_norm(x, (d,), P["norm.weight"], eps)
    head = P["tok_embeddings.weight"] if tied else P["lm_head.weight"]
    logits = F.linear(x, head).reshape(B * S, vocab)
    loss = F.cross_entropy(logits, tgt_t, ignore_index=-100)
    if aux_total is not None:
        loss = loss + aux_total
    loss.backward()
    params = [P[name] for name, _ in lay]
    norm = torch.nn.utils.clip_grad_norm_(params, max_grad_norm)
    grads = np.concatenate([P[name].grad.detach().numpy().reshape(-1) for name, _ in lay])
    opt = torch.optim.AdamW(params, lr=lr, betas=betas, eps=adam_eps, weight_decay=weight_decay)
    opt.step()
    new_params = np.concatenate([P[name].detach().numpy().reshape(-1) for name, _ in lay])
    return float(loss), float(norm), grads, new_params


# ----------------------------------------------------------------------------- mixture of experts
def moe_topk(logits, k):
    """Top-k expert indices per row: larger logit first, ties to the lower index (numpy)."""
    T, E = logits.shape
    order = np.lexsort((np.broadcast_to(np.arange(E), (T, E)), -logits.astype(np.float64)), axis=1)
    return order[:, :k].astype(np.int64)


def moe_layer(th, twr, experts, k, aux_coef):
    """The MoE layer as a torch graph (src/nn/moe.cpp:33-253): th [T, d], router twr [E, d],
    experts [(gate, up, down)] -> (y [T, d], aux).  Every active expert runs on all tokens,
    weighted by the normalised masked gate; aux uses route()'s own softmax."""
    T, d = th.shape
    E = twr.shape[0]
    logits = th @ twr.T
    idx = torch.tensor(moe_topk(logits.detach().numpy(), k))
    probs_r = torch.softmax(th @ twr.T, dim=-1)
    counts = torch.bincount(idx.reshape(-1), minlength=E).to(th.dtype)
    f_e = counts * (E * aux_coef) / (T * k)
    aux = (probs_r.mean(0) * f_e).sum() if (aux_coef > 0 and E > 1) else torch.zeros((), dtype=th.dtype)
    probs = torch.softmax(logits, dim=-1)
    mask = torch.zeros(T, E, dtype=th.dtype)
    mask.scatter_(1, idx, 1.0)
    masked = probs * mask
    gates = masked / (masked.sum(-1, keepdim=True) + 1e-9)
    y = torch.zeros(T, d, dtype=th.dtype)
    for e in range(E):
        if counts[e] == 0:
            continue
        wg, wu, wd = experts[e]
        a = F.silu(th @ wg.T) * (th @ wu.T)
        y = y + (a @ wd.T) * gates[:, e:e + 1]
    return y, aux


def moe_ffn_torch(h, wr, wg, wu, wd, k, aux_coef, dy=None, daux=1.0):
    """float64 MoE layer (moe_layer) on numpy inputs.  Returns y, aux and, when dy is given, the
    gradients of sum(y * dy) + daux * aux wrt (h, wr, wg, wu, wd)."""
    t = [torch.tensor(np.asarray(a, np.float64), requires_grad=True) for a in (h, wr, wg, wu, wd)]
    th, twr, twg, twu, twd = t
    y, aux = moe_layer(th, twr, [(twg[e], twu[e], twd[e]) for e in range(twr.shape[0])], k, aux_coef)
    out = [y.detach().numpy(), float(aux.detach())]
    if dy is not None:
        loss = (y * torch.tensor(np.asarray(dy, np.float64))).sum() + daux * aux
        loss.backward()
        out.append([None if x.grad is None else x.grad.numpy() for x in t])
    return out
