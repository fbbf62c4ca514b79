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


def layout(vocab, d, n_layers, f, tied):
    """(name, shape) in the flat order the oracle and the product arena share."""
    out = [("tok_embeddings.weight", (vocab, d))]
    for l in range(n_layers):
        p = f"layers.{l}."
        out += [(p + "attn.q_proj.weight", (d, d)), (p + "attn.k_proj.weight", (d, d)),
                (p + "attn.v_proj.weight", (d, d)), (p + "attn.out_proj.weight", (d, d)),
                (p + "ffn.gate_proj.weight", (f, d)), (p + "ffn.up_proj.weight", (f, d)),
                (p + "ffn.down_proj.weight", (d, f)), (p + "norm1.weight", (d,)), (p + "norm2.weight", (d,))]
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
            betas=(0.9, 0.95), adam_eps=1e-8, weight_decay=0.1, max_grad_norm=1.0, dtype=torch.float64):
    lay = layout(vocab, d, n_layers, f, tied)
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
        a = F.silu(F.linear(h, P[p + "ffn.gate_proj.weight"])) * F.linear(h, P[p + "ffn.up_proj.weight"])
        x = x + F.linear(a, P[p + "ffn.down_proj.weight"])
    x = F.rms_norm(x, (d,), P["norm.weight"], eps)
    head = P["tok_embeddings.weight"] if tied else P["lm_head.weight"]
    logits = F.linear(x, head).reshape(B * S, vocab)
    loss = F.cross_entropy(logits, tgt_t, ignore_index=-100)
    loss.backward()
    params = [P[name] for name, _ in lay]
    norm = torch.nn.utils.clip_grad_norm_(params, max_grad_norm)
    grads = np.concatenate([P[name].grad.detach().numpy().reshape(-1) for name, _ in lay])
    opt = torch.optim.AdamW(params, lr=lr, betas=betas, eps=adam_eps, weight_decay=weight_decay)
    opt.step()
    new_params = np.concatenate([P[name].detach().numpy().reshape(-1) for name, _ in lay])
    return float(loss), float(norm), grads, new_params
