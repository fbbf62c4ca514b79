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


PROJ = ("attn.q_proj", "attn.k_proj", "attn.v_proj", "attn.out_proj", "ffn.gate_proj", "ffn.up_proj",
        "ffn.down_proj")


def lora_layout(d, n_layers, f, r):
    """(name, shape) of the LoRA adapters in the packed order of the trainable arena."""
    out = []
    for l in range(n_layers):
        p = f"layers.{l}."
        out += [(p + "attn.q_proj.lora_A", (r, d)), (p + "attn.k_proj.lora_A", (r, d)),
                (p + "attn.v_proj.lora_A", (r, d)), (p + "attn.q_proj.lora_B", (d, r)),
                (p + "attn.k_proj.lora_B", (d, r)), (p + "attn.v_proj.lora_B", (d, r)),
                (p + "attn.out_proj.lora_A", (r, d)), (p + "attn.out_proj.lora_B", (d, r)),
                (p + "ffn.gate_proj.lora_A", (r, d)), (p + "ffn.up_proj.lora_A", (r, d)),
                (p + "ffn.gate_proj.lora_B", (f, r)), (p + "ffn.up_proj.lora_B", (f, r)),
                (p + "ffn.down_proj.lora_A", (r, f)), (p + "ffn.down_proj.lora_B", (d, r))]
    return out


def int4_round_trip(w, G):
    """INT4-symmetric quantize + dequantize of a flat float32 array in groups of G, fp16 scales
    (numpy): s = max(absmax / 7, 1e-8) in float32, q = clamp(round half away(w / s), -7, 7),
    w' = q * float(fp16(s))."""
    w = np.asarray(w, np.float32).reshape(-1, G)
    s = np.maximum(np.abs(w).max(axis=1) / np.float32(7.0), np.float32(1e-8)).astype(np.float32)
    v = (w / s[:, None]).astype(np.float64)
    q = np.clip(np.sign(v) * np.floor(np.abs(v) + 0.5), -7, 7)
    s16 = s.astype(np.float16).astype(np.float32)
    return (q.astype(np.float32) * s16[:, None]).reshape(-1)


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
            n_experts=0, top_k=2, aux_coef=0.01, lora=None, moe_forced=None):
    """Returns loss (cross-entropy + the MoE aux losses), pre-clip grad norm, grads, updated params.
    lora = (lora_flat, r, alpha, G): params_flat is the frozen base, its projections enter as their
    INT4 round trip, and the LoRA adapters (y += (x A^T) B^T * alpha / r) are the trained tensors.
    moe_forced ([n_layers, B*S, top_k]): each MoE layer's top-k selection instead of its router's."""
    lay = layout(vocab, d, n_layers, f, tied, n_experts)
    P = {}
    off = 0
    for name, shape in lay:
        n = int(np.prod(shape))
        w = params_flat[off:off + n]
        if lora is not None and any(pr + ".weight" in name for pr in PROJ):
            w = int4_round_trip(w, lora[3])
        P[name] = torch.tensor(w.reshape(shape), dtype=dtype, requires_grad=lora is None)
        off += n
    assert off == params_flat.size
    if lora is not None:
        lay_t = lora_layout(d, n_layers, f, lora[1])
        off = 0
        for name, shape in lay_t:
            n = int(np.prod(shape))
            P[name] = torch.tensor(lora[0][off:off + n].reshape(shape), dtype=dtype, requires_grad=True)
            off += n
        assert off == lora[0].size
        scaling = lora[2] / lora[1]
    else:
        lay_t = lay

    def lin(x, pre):
        y = F.linear(x, P[pre + ".weight"])
        if lora is not None:
            y = y + F.linear(F.linear(x, P[pre + ".lora_A"]), P[pre + ".lora_B"]) * scaling
        return y

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
        q = lin(h, p + "attn.q_proj").view(B, S, n_heads, hd).transpose(1, 2)
        k = lin(h, p + "attn.k_proj").view(B, S, n_heads, hd).transpose(1, 2)
        v = lin(h, p + "attn.v_proj").view(B, S, n_heads, hd).transpose(1, 2)
        q, k = rope(q, cos, sin), rope(k, cos, sin)
        o = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        o = o.transpose(1, 2).reshape(B, S, d)
        x = x + lin(o, p + "attn.out_proj")
        h = F.rms_norm(x, (d,), P[p + "norm2.weight"], eps)
        if n_experts:
            ex = [(P[p + f"moe.experts.{e}.gate_proj.weight"], P[p + f"moe.experts.{e}.up_proj.weight"],
                   P[p + f"moe.experts.{e}.down_proj.weight"]) for e in range(n_experts)]
            y, aux = moe_layer(h.reshape(B * S, d), P[p + "moe.router.gate.weight"], ex, top_k, aux_coef,
                               None if moe_forced is None else moe_forced[l])
            x = x + y.reshape(B, S, d)
            aux_total = aux if aux_total is None else aux_total + aux
        else:
            a = F.silu(lin(h, p + "ffn.gate_proj")) * lin(h, p + "ffn.up_proj")
            x = x + lin(a, p + "ffn.down_proj")
    x = F.rms_norm(x, (d,), P["norm.weight"], eps)
    head = P["tok_embeddings.weight"] if tied else P["lm_head.weight"]
    logits = F.linear(x, head).reshape(B * S, vocab)
    loss = F.cross_entropy(logits, tgt_t, ignore_index=-100)
    if aux_total is not None:
        loss = loss + aux_total
    loss.backward()
    params = [P[name] for name, _ in lay_t]
    norm = torch.nn.utils.clip_grad_norm_(params, max_grad_norm)
    grads = np.concatenate([P[name].grad.detach().numpy().reshape(-1) for name, _ in lay_t])
    opt = torch.optim.AdamW(params, lr=lr, betas=betas, eps=adam_eps, weight_decay=weight_decay)
    opt.step()
    new_params = np.concatenate([P[name].detach().numpy().reshape(-1) for name, _ in lay_t])
    return float(loss.detach()), float(norm), grads, new_params


# ----------------------------------------------------------------------------- mixture of experts
def moe_topk(logits, k):
    """Top-k expert indices per row: larger logit first, ties to the lower index (numpy)."""
    T, E = logits.shape
    order = np.lexsort((np.broadcast_to(np.arange(E), (T, E)), -logits.astype(np.float64)), axis=1)
    return order[:, :k].astype(np.int64)


def moe_layer(th, twr, experts, k, aux_coef, forced=None):
    """The MoE layer as a torch graph (src/nn/moe.cpp:33-253): th [T, d], router twr [E, d],
    experts [(gate, up, down)] -> (y [T, d], aux).  Every active expert runs on all tokens,
    weighted by the normalised masked gate; aux uses route()'s own softmax."""
    T, d = th.shape
    E = twr.shape[0]
    logits = th @ twr.T
    idx = torch.tensor(moe_topk(logits.detach().numpy(), k) if forced is None else np.asarray(forced, np.int64))
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
