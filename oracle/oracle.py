"""ctypes front end of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker or the timed CPU baseline.  The product
package never imports it.  Each wrapper names the C function it calls; the C functions
cite the reference file:line they restate.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

f32p = C.POINTER(C.c_float)
i64p = C.POINTER(C.c_int64)


class LMConfig(C.Structure):
    _fields_ = [("vocab", C.c_int64), ("d_model", C.c_int64), ("n_layers", C.c_int64),
                ("n_heads", C.c_int64), ("d_ffn", C.c_int64), ("max_seq_len", C.c_int64),
                ("norm_eps", C.c_float), ("rope_base", C.c_float), ("tied", C.c_int), ("n_experts", C.c_int64),
                ("top_k", C.c_int64), ("aux_coef", C.c_float)]


class TrainOpts(C.Structure):
    _fields_ = [("lr", C.c_float), ("beta1", C.c_float), ("beta2", C.c_float), ("eps", C.c_float),
                ("weight_decay", C.c_float), ("max_grad_norm", C.c_float), ("use_scaler", C.c_int),
                ("do_update", C.c_int)]


class StepResult(C.Structure):
    _fields_ = [("loss", C.c_float), ("grad_norm", C.c_float), ("found_inf", C.c_int),
                ("loss_scale_used", C.c_float), ("t_embed", C.c_double), ("t_blocks_fwd", C.c_double),
                ("t_head_fwd", C.c_double), ("t_loss", C.c_double), ("t_head_bwd", C.c_double),
                ("t_blocks_bwd", C.c_double), ("t_embed_bwd", C.c_double), ("t_optim", C.c_double),
                ("aux_loss", C.c_float)]


class Scaler(C.Structure):
    _fields_ = [("initial_scale", C.c_float), ("growth_factor", C.c_float), ("backoff_factor", C.c_float),
                ("growth_interval", C.c_int), ("min_scale", C.c_float), ("max_scale", C.c_float),
                ("scale", C.c_float), ("good_steps", C.c_int), ("skipped_steps", C.c_int)]


def build() -> str:
    """Compile liboracle.so with oracle/Makefile (gcc, AVX2+FMA)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        L.orc_ce_fwd.restype = C.c_float
        L.orc_ce_fwd_soft.restype = C.c_float
        L.orc_clip_grad_norm.restype = C.c_float
        L.orc_lm_loss.restype = C.c_float
        L.orc_lm_num_params.restype = C.c_int64
        L.orc_qlora_num_params.restype = C.c_int64
        L.orc_get_threads.restype = C.c_int
        _lib = L
    return _lib


def _f(a):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(f32p)


def _i(a):
    assert a.dtype == np.int64 and a.flags.c_contiguous
    return a.ctypes.data_as(i64p)


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


def threads() -> int:
    return lib().orc_get_threads()


def gemm(A, B):
    """orc_gemm: C = A @ B (fp32, reference AVX2 microkernel order)."""
    A = np.ascontiguousarray(A, np.float32)
    B = np.ascontiguousarray(B, np.float32)
    M, K = A.shape
    K2, N = B.shape
    assert K == K2
    Cm = np.empty((M, N), np.float32)
    lib().orc_gemm(_f(A), _f(B), _f(Cm), C.c_int64(M), C.c_int64(N), C.c_int64(K))
    return Cm


def linear_fwd(x, W, B, S):
    x = np.ascontiguousarray(x, np.float32)
    W = np.ascontiguousarray(W, np.float32)
    out, inn = W.shape
    y = np.empty((B * S, out), np.float32)
    lib().orc_linear_fwd(_f(x), _f(W), _f(y), C.c_int64(B), C.c_int64(S), C.c_int64(inn), C.c_int64(out))
    return y


def linear_bwd(x, W, dy, B, S):
    x = np.ascontiguousarray(x, np.float32)
    W = np.ascontiguousarray(W, np.float32)
    dy = np.ascontiguousarray(dy, np.float32)
    out, inn = W.shape
    dx = np.empty((B * S, inn), np.float32)
    dW = np.zeros((out, inn), np.float32)
    lib().orc_linear_bwd(_f(x), _f(W), _f(dy), _f(dx), _f(dW), C.c_int64(B), C.c_int64(S), C.c_int64(inn),
                         C.c_int64(out))
    return dx, dW


def rmsnorm_fwd(x, w, eps):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    rows, d = x.shape
    y = np.empty_like(x)
    rms = np.empty(rows, np.float32)
    lib().orc_rmsnorm_fwd(_f(x), _f(w), _f(y), _f(rms), C.c_int64(rows), C.c_int64(d), C.c_float(eps))
    return y, rms


def rmsnorm_bwd(dy, x, w, rms):
    dy = np.ascontiguousarray(dy, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    rows, d = x.shape
    dx = np.empty_like(x)
    dw = np.zeros(d, np.float32)
    lib().orc_rmsnorm_bwd(_f(dy), _f(x), _f(np.ascontiguousarray(w, np.float32)), _f(rms), _f(dx), _f(dw),
                          C.c_int64(rows), C.c_int64(d))
    return dx, dw


def rope_tables(max_seq, hd, base=10000.0):
    c = np.empty((max_seq, hd // 2), np.float32)
    s = np.empty((max_seq, hd // 2), np.float32)
    lib().orc_rope_tables(_f(c), _f(s), C.c_int64(max_seq), C.c_int64(hd), C.c_float(base))
    return c, s


def rope_fwd(x, B, S, H, hd, start_pos=0, base=10000.0):
    """x: [B*S, H*hd]; returns the rotated copy."""
    x = np.array(x, np.float32, copy=True, order="C")
    c, s = rope_tables(start_pos + S, hd, base)
    lib().orc_rope_fwd(_f(x), _f(c), _f(s), C.c_int64(B), C.c_int64(S), C.c_int64(H), C.c_int64(hd),
                       C.c_int64(start_pos))
    return x


def rope_bwd(g, B, S, H, hd, start_pos=0, base=10000.0):
    g = np.array(g, np.float32, copy=True, order="C")
    c, s = rope_tables(start_pos + S, hd, base)
    lib().orc_rope_bwd(_f(g), _f(c), _f(s), C.c_int64(B), C.c_int64(S), C.c_int64(H), C.c_int64(hd),
                       C.c_int64(start_pos))
    return g


def attention_fwd(q, k, v, B, S, H, hd, causal=True, keep=True):
    """q,k,v: [B*S, H*hd] (= [B,S,H,hd]).  Returns o and (E, rowsum) for the backward."""
    q, k, v = (np.ascontiguousarray(t, np.float32) for t in (q, k, v))
    o = np.empty_like(q)
    E = np.empty((B, H, S, S), np.float32) if keep else None
    rs = np.empty((B, H, S), np.float32) if keep else None
    lib().orc_attention_fwd(_f(q), _f(k), _f(v), _f(o), _f(E) if keep else None, _f(rs) if keep else None,
                            C.c_int64(B), C.c_int64(S), C.c_int64(H), C.c_int64(hd), C.c_int(1 if causal else 0))
    return o, E, rs


def attention_bwd(q, k, v, E, rs, do, B, S, H, hd):
    q, k, v, do = (np.ascontiguousarray(t, np.float32) for t in (q, k, v, do))
    dq, dk, dv = np.empty_like(q), np.empty_like(k), np.empty_like(v)
    lib().orc_attention_bwd(_f(q), _f(k), _f(v), _f(E), _f(rs), _f(do), _f(dq), _f(dk), _f(dv),
                            C.c_int64(B), C.c_int64(S), C.c_int64(H), C.c_int64(hd))
    return dq, dk, dv


def swiglu_fwd(g, u):
    g = np.ascontiguousarray(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    h = np.empty_like(g)
    lib().orc_swiglu_fwd(_f(g), _f(u), _f(h), C.c_int64(g.size))
    return h


def swiglu_bwd(g, u, dh):
    g, u, dh = (np.ascontiguousarray(t, np.float32) for t in (g, u, dh))
    dg, du = np.empty_like(g), np.empty_like(u)
    lib().orc_swiglu_bwd(_f(g), _f(u), _f(dh), _f(dg), _f(du), C.c_int64(g.size))
    return dg, du


def ce_fwd(logits, targets, ignore_index=-100):
    logits = np.ascontiguousarray(logits, np.float32)
    targets = np.ascontiguousarray(targets, np.int64)
    N, Cn = logits.shape
    losses = np.empty(N, np.float32)
    lse = np.empty(N, np.float32)
    valid = C.c_int64(0)
    loss = lib().orc_ce_fwd(_f(logits), _i(targets), C.c_int64(N), C.c_int64(Cn), C.c_int64(ignore_index),
                            _f(losses), _f(lse), C.byref(valid))
    return float(loss), losses, lse, int(valid.value)


def ce_bwd(logits, targets, lse, valid, g=1.0, ignore_index=-100):
    logits = np.ascontiguousarray(logits, np.float32)
    targets = np.ascontiguousarray(targets, np.int64)
    N, Cn = logits.shape
    d = np.empty_like(logits)
    lib().orc_ce_bwd(_f(logits), _i(targets), _f(np.ascontiguousarray(lse, np.float32)), C.c_int64(N),
                     C.c_int64(Cn), C.c_int64(ignore_index), C.c_int64(valid), C.c_float(g), _f(d))
    return d


CE_REDUCTIONS = {"mean": 0, "sum": 1, "none": 2}


def flash_fwd(q, k, v, causal=True, scale=None):
    """orc_flash_fwd on [BH, Sq, D] / [BH, Sk, D] arrays: (o, lse)."""
    q, k, v = (np.ascontiguousarray(x, np.float32) for x in (q, k, v))
    BH, Sq, D = q.shape
    Sk = k.shape[1]
    assert k.shape == (BH, Sk, D) and v.shape == k.shape
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    o = np.empty_like(q)
    lse = np.empty((BH, Sq), np.float32)
    lib().orc_flash_fwd(_f(q), _f(k), _f(v), _f(o), _f(lse), C.c_int64(BH), C.c_int64(Sq), C.c_int64(Sk),
                        C.c_int64(D), C.c_int(1 if causal else 0), C.c_float(scale))
    return o, lse


def flash_bwd(q, k, v, o, do, lse, causal=True, scale=None):
    """orc_flash_bwd: (dq, dk, dv)."""
    q, k, v, o, do = (np.ascontiguousarray(x, np.float32) for x in (q, k, v, o, do))
    BH, Sq, D = q.shape
    Sk = k.shape[1]
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    lib().orc_flash_bwd(_f(q), _f(k), _f(v), _f(o), _f(do), _f(np.ascontiguousarray(lse, np.float32)), _f(dq),
                        _f(dk), _f(dv), C.c_int64(BH), C.c_int64(Sq), C.c_int64(Sk), C.c_int64(D),
                        C.c_int(1 if causal else 0), C.c_float(scale))
    return dq, dk, dv


def ce_fwd_soft(logits, y):
    """orc_ce_fwd_soft: (mean loss, per-row losses, lse) for distribution targets y [N, C]."""
    logits = np.ascontiguousarray(logits, np.float32)
    y = np.ascontiguousarray(y, np.float32)
    N, Cn = logits.shape
    assert y.shape == logits.shape
    losses = np.empty(N, np.float32)
    lse = np.empty(N, np.float32)
    mean = lib().orc_ce_fwd_soft(_f(logits), _f(y), C.c_int64(N), C.c_int64(Cn), _f(losses), _f(lse))
    return float(mean), losses, lse


def ce_bwd_soft(logits, y, lse, g=None, per_row=False, divisor=1.0):
    """orc_ce_bwd_soft: (softmax - y) * scale; g None (1), a scalar or per-row values."""
    logits = np.ascontiguousarray(logits, np.float32)
    y = np.ascontiguousarray(y, np.float32)
    N, Cn = logits.shape
    d = np.empty_like(logits)
    gp = None if g is None else np.ascontiguousarray(np.atleast_1d(g), np.float32)
    lib().orc_ce_bwd_soft(_f(logits), _f(y), _f(np.ascontiguousarray(lse, np.float32)), C.c_int64(N), C.c_int64(Cn),
                          None if gp is None else _f(gp), C.c_int(1 if per_row else 0), C.c_float(divisor), _f(d))
    return d


def ce_bwd_reduction(logits, targets, lse, valid, reduction, g=None, ignore_index=-100):
    """orc_ce_bwd_reduction: g None (1), a scalar ("mean"/"sum") or per-row values ("none")."""
    logits = np.ascontiguousarray(logits, np.float32)
    targets = np.ascontiguousarray(targets, np.int64)
    N, Cn = logits.shape
    d = np.empty_like(logits)
    gp = None if g is None else np.ascontiguousarray(np.atleast_1d(g), np.float32)
    lib().orc_ce_bwd_reduction(_f(logits), _i(targets), _f(np.ascontiguousarray(lse, np.float32)), C.c_int64(N),
                               C.c_int64(Cn), C.c_int64(ignore_index), C.c_int(CE_REDUCTIONS[reduction]),
                               C.c_int64(valid), _f(gp) if gp is not None else None, _f(d))
    return d


def embedding_fwd(ids, W):
    ids = np.ascontiguousarray(ids, np.int64).reshape(-1)
    W = np.ascontiguousarray(W, np.float32)
    V, D = W.shape
    out = np.empty((ids.size, D), np.float32)
    lib().orc_embedding_fwd(_i(ids), _f(W), _f(out), C.c_int64(ids.size), C.c_int64(D), C.c_int64(V))
    return out


def embedding_bwd(ids, dout, V):
    ids = np.ascontiguousarray(ids, np.int64).reshape(-1)
    dout = np.ascontiguousarray(dout, np.float32)
    D = dout.shape[1]
    dW = np.zeros((V, D), np.float32)
    lib().orc_embedding_bwd(_i(ids), _f(dout), _f(dW), C.c_int64(ids.size), C.c_int64(D), C.c_int64(V))
    return dW


def adamw(p, g, m, v, lr, beta1, beta2, eps, wd, step):
    """In place on p, m, v (float32 arrays)."""
    lib().orc_adamw(_f(p), _f(g), _f(m), _f(v), C.c_int64(p.size), C.c_float(lr), C.c_float(beta1),
                    C.c_float(beta2), C.c_float(eps), C.c_float(wd), C.c_int64(step))


def clip_grad_norm(grads, max_norm):
    """In place on the list of float32 arrays; returns the pre-clip norm."""
    n = len(grads)
    ptrs = (f32p * n)(*[_f(g) for g in grads])
    sizes = (C.c_int64 * n)(*[g.size for g in grads])
    return float(lib().orc_clip_grad_norm(ptrs, sizes, C.c_int64(n), C.c_float(max_norm)))


class LossScaler:
    """orc_scaler_*: the reference DynamicLossScaler state machine."""

    def __init__(self, initial_scale=65536.0, growth_factor=2.0, backoff_factor=0.5, growth_interval=1000,
                 min_scale=1.0, max_scale=16777216.0):
        self.s = Scaler()
        lib().orc_scaler_init(C.byref(self.s), C.c_float(initial_scale), C.c_float(growth_factor),
                              C.c_float(backoff_factor), C.c_int(growth_interval), C.c_float(min_scale),
                              C.c_float(max_scale))

    def unscale_and_update(self, grads):
        n = len(grads)
        ptrs = (f32p * n)(*[_f(g) for g in grads])
        sizes = (C.c_int64 * n)(*[g.size for g in grads])
        return bool(lib().orc_scaler_unscale_and_update(C.byref(self.s), ptrs, sizes, C.c_int64(n)))

    @property
    def scale(self):
        return self.s.scale

    @property
    def good_steps(self):
        return self.s.good_steps

    @property
    def skipped_steps(self):
        return self.s.skipped_steps


def make_config(vocab, d_model, n_layers, n_heads, d_ffn, max_seq_len, norm_eps=1e-6, rope_base=10000.0,
                tied=False, n_experts=0, top_k=2, aux_coef=0.01):
    return LMConfig(vocab, d_model, n_layers, n_heads, d_ffn, max_seq_len, norm_eps, rope_base, 1 if tied else 0,
                    n_experts, top_k, aux_coef)


def num_params(cfg: LMConfig) -> int:
    return int(lib().orc_lm_num_params(C.byref(cfg)))


def lm_loss(cfg, params, ids, targets, B, S):
    return float(lib().orc_lm_loss(C.byref(cfg), _f(params), _i(np.ascontiguousarray(ids, np.int64)),
                                   _i(np.ascontiguousarray(targets, np.int64)), C.c_int64(B), C.c_int64(S)))


def lm_logits(cfg, params, ids, B, S):
    out = np.empty((B * S, cfg.vocab), np.float32)
    rc = lib().orc_lm_logits(C.byref(cfg), _f(np.ascontiguousarray(params, np.float32)),
                             _i(np.ascontiguousarray(ids, np.int64)), C.c_int64(B), C.c_int64(S), _f(out))
    if rc != 0:
        raise RuntimeError(f"orc_lm_logits failed with {rc}")
    return out.reshape(B, S, cfg.vocab)


def lm_step(cfg, params, ids, targets, B, S, lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1,
            max_grad_norm=1.0, m=None, v=None, step=0, scaler: LossScaler | None = None, do_update=True,
            moe_forced=None, moe_route_out=None):
    """One training step in place on `params` (float32 flat).  Returns (result, grads, m, v, step).
    MoE configurations: moe_forced ([n_layers, T, top_k] int64) makes every layer use that top-k
    selection instead of its router's; moe_route_out (same shape, int64, written) receives the
    selections the forward used (orc_moe_set_routing)."""
    if moe_forced is not None or moe_route_out is not None:
        shape = (cfg.n_layers, B * S, cfg.top_k)
        forced = None if moe_forced is None else np.ascontiguousarray(moe_forced, np.int64).reshape(shape)
        if moe_route_out is not None:
            assert moe_route_out.dtype == np.int64 and moe_route_out.flags.c_contiguous and moe_route_out.size == np.prod(shape)
        lib().orc_moe_set_routing(_i(forced) if forced is not None else None,
                                  _i(moe_route_out) if moe_route_out is not None else None)
        try:
            return lm_step(cfg, params, ids, targets, B, S, lr, beta1, beta2, eps, weight_decay, max_grad_norm, m, v,
                           step, scaler, do_update)
        finally:
            lib().orc_moe_set_routing(None, None)
    n = num_params(cfg)
    assert params.size == n and params.dtype == np.float32
    grads = np.zeros(n, np.float32)
    m = np.zeros(n, np.float32) if m is None else m
    v = np.zeros(n, np.float32) if v is None else v
    stepc = C.c_int64(step)
    opts = TrainOpts(lr, beta1, beta2, eps, weight_decay, max_grad_norm, 1 if scaler else 0, 1 if do_update else 0)
    res = StepResult()
    rc = lib().orc_lm_step(C.byref(cfg), _f(params), _f(grads), _f(m), _f(v), C.byref(stepc),
                           _i(np.ascontiguousarray(ids, np.int64)), _i(np.ascontiguousarray(targets, np.int64)),
                           C.c_int64(B), C.c_int64(S), C.byref(opts), C.byref(scaler.s) if scaler else None,
                           C.byref(res))
    if rc != 0:
        raise RuntimeError(f"orc_lm_step failed with {rc}")
    return res, grads, m, v, int(stepc.value)


def qlora_num_params(cfg: LMConfig, r: int) -> int:
    return int(lib().orc_qlora_num_params(C.byref(cfg), C.c_int64(r)))


def qlora_dequantize_base(cfg, G, params):
    """The dense parameters with every layer's seven projections replaced by their INT4 round trip
    (groups of G, fp16 scales)."""
    out = np.ascontiguousarray(params, np.float32).copy()
    rc = lib().orc_qlora_dequantize_base(C.byref(cfg), C.c_int64(G), _f(out))
    if rc != 0:
        raise RuntimeError(f"orc_qlora_dequantize_base failed with {rc}")
    return out


def qlora_step(cfg, r, alpha, G, base, lora, ids, targets, B, S, lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8,
               weight_decay=0.1, max_grad_norm=1.0, m=None, v=None, step=0, scaler: LossScaler | None = None,
               do_update=True):
    """One QLoRA step in place on `lora` (float32 flat adapters); base is frozen.
    Returns (result, grads, m, v, step)."""
    n = qlora_num_params(cfg, r)
    assert lora.size == n and lora.dtype == np.float32
    base = np.ascontiguousarray(base, np.float32)
    assert base.size == num_params(cfg)
    grads = np.zeros(n, np.float32)
    m = np.zeros(n, np.float32) if m is None else m
    v = np.zeros(n, np.float32) if v is None else v
    stepc = C.c_int64(step)
    opts = TrainOpts(lr, beta1, beta2, eps, weight_decay, max_grad_norm, 1 if scaler else 0, 1 if do_update else 0)
    res = StepResult()
    rc = lib().orc_qlora_step(C.byref(cfg), C.c_int64(r), C.c_float(alpha), C.c_int64(G), _f(base), _f(lora),
                              _f(grads), _f(m), _f(v), C.byref(stepc), _i(np.ascontiguousarray(ids, np.int64)),
                              _i(np.ascontiguousarray(targets, np.int64)), C.c_int64(B), C.c_int64(S),
                              C.byref(opts), C.byref(scaler.s) if scaler else None, C.byref(res))
    if rc != 0:
        raise RuntimeError(f"orc_qlora_step failed with {rc}")
    return res, grads, m, v, int(stepc.value)


# ----------------------------------------------------------------------------- mixture of experts
def moe_route(logits, k, aux_coef):
    """orc_moe_route: returns idx [T,k] int64, rweights [T,k], gates [T,E], probs [T,E],
    counts [E] int64, mean_probs [E], aux (float)."""
    logits = np.ascontiguousarray(logits, np.float32)
    T, E = logits.shape
    assert E <= 256
    idx = np.empty((T, k), np.int64)
    rw = np.empty((T, k), np.float32)
    gates = np.empty((T, E), np.float32)
    probs = np.empty((T, E), np.float32)
    counts = np.empty(E, np.int64)
    mp = np.empty(E, np.float32)
    aux = C.c_float(0.0)
    lib().orc_moe_route(_f(logits), C.c_int64(T), C.c_int64(E), C.c_int64(k), C.c_float(aux_coef), _i(idx), _f(rw),
                        _f(gates), _f(probs), _i(counts), _f(mp), C.byref(aux))
    return idx, rw, gates, probs, counts, mp, aux.value


def moe_ffn_fwd(h, wr, wg, wu, wd, k, aux_coef):
    """orc_moe_ffn_fwd: h [T,d], wr [E,d], wg/wu [E,f,d], wd [E,d,f] -> y [T,d], aux, idx, gates."""
    h, wr, wg, wu, wd = (np.ascontiguousarray(t, np.float32) for t in (h, wr, wg, wu, wd))
    T, d = h.shape
    E, f, _ = wg.shape
    assert E <= 256
    y = np.empty((T, d), np.float32)
    idx = np.empty((T, k), np.int64)
    gates = np.empty((T, E), np.float32)
    aux = C.c_float(0.0)
    lib().orc_moe_ffn_fwd(_f(h), _f(wr), _f(wg), _f(wu), _f(wd), C.c_int64(T), C.c_int64(d), C.c_int64(f),
                          C.c_int64(E), C.c_int64(k), C.c_float(aux_coef), _f(y), C.byref(aux), _i(idx), _f(gates))
    return y, aux.value, idx, gates


def moe_ffn_bwd(h, wr, wg, wu, wd, k, aux_coef, dy, daux):
    """orc_moe_ffn_bwd: returns dh, dwr, dwg, dwu, dwd for dL/dy = dy and dL/daux = daux."""
    h, wr, wg, wu, wd, dy = (np.ascontiguousarray(t, np.float32) for t in (h, wr, wg, wu, wd, dy))
    T, d = h.shape
    E, f, _ = wg.shape
    dh = np.zeros((T, d), np.float32)
    dwr = np.zeros_like(wr)
    dwg = np.zeros_like(wg)
    dwu = np.zeros_like(wu)
    dwd = np.zeros_like(wd)
    lib().orc_moe_ffn_bwd(_f(h), _f(wr), _f(wg), _f(wu), _f(wd), C.c_int64(T), C.c_int64(d), C.c_int64(f),
                          C.c_int64(E), C.c_int64(k), C.c_float(aux_coef), _f(dy), C.c_float(daux), _f(dh), _f(dwr),
                          _f(dwg), _f(dwu), _f(dwd))
    return dh, dwr, dwg, dwu, dwd


# ----------------------------------------------------------------------------- INT4 + LoRA
def f32_to_f16_bits(x):
    """orc_f32_to_f16 over an array: uint16 bits of fp16(x), round to nearest even."""
    L = lib()
    L.orc_f32_to_f16.restype = C.c_uint16
    L.orc_f32_to_f16.argtypes = [C.c_float]
    x = np.asarray(x, np.float32).ravel()
    return np.array([L.orc_f32_to_f16(float(v)) for v in x], np.uint16)


def int4_quantize(x, G, scale_f16=False):
    """orc_int4_quantize of the flat x: returns packed uint8 [(n+1)/2] and scales
    (float32, or float16 when scale_f16) [ceil(n/G)]."""
    x = np.ascontiguousarray(x, np.float32).ravel()
    n = x.size
    g = n if (G <= 0 or G > n) else G
    ng = (n + g - 1) // g if n else 0
    packed = np.zeros((n + 1) // 2, np.uint8)
    scales = np.zeros(ng, np.float16 if scale_f16 else np.float32)
    rc = lib().orc_int4_quantize(_f(x), C.c_int64(n), C.c_int64(G), C.c_int(1 if scale_f16 else 0),
                                 packed.ctypes.data_as(C.c_void_p), scales.ctypes.data_as(C.c_void_p))
    if rc != 0:
        raise ValueError(f"orc_int4_quantize failed with {rc}")
    return packed, scales


def int4_dequantize(packed, scales, n, G):
    """orc_int4_dequantize: float32 [n]; scales may be float32 or float16."""
    packed = np.ascontiguousarray(packed, np.uint8)
    scales = np.ascontiguousarray(scales)
    out = np.empty(n, np.float32)
    rc = lib().orc_int4_dequantize(packed.ctypes.data_as(C.c_void_p), scales.ctypes.data_as(C.c_void_p),
                                   C.c_int(1 if scales.dtype == np.float16 else 0), C.c_int64(n), C.c_int64(G),
                                   _f(out))
    if rc != 0:
        raise ValueError(f"orc_int4_dequantize failed with {rc}")
    return out


def int4_dequantize_zp(packed, scales, zp, is_signed, n, G):
    """orc_int4_dequantize_zp: float32 [n]; fp32 scales and zero points (zp None: none)."""
    packed = np.ascontiguousarray(packed, np.uint8)
    scales = np.ascontiguousarray(scales, np.float32)
    zpa = None if zp is None else np.ascontiguousarray(zp, np.float32)
    out = np.empty(n, np.float32)
    rc = lib().orc_int4_dequantize_zp(packed.ctypes.data_as(C.c_void_p), _f(scales),
                                      None if zpa is None else _f(zpa), C.c_int(1 if is_signed else 0),
                                      C.c_int64(n), C.c_int64(G), _f(out))
    if rc != 0:
        raise ValueError(f"orc_int4_dequantize_zp failed with {rc}")
    return out


def lora_fwd(x, W, A, Bm, scaling, Bt, S):
    """orc_lora_fwd: x [Bt*S,in], W [out,in], A [r,in], Bm [out,r] -> y [Bt*S,out], xa [Bt*S,r]."""
    x, W, A, Bm = (np.ascontiguousarray(t, np.float32) for t in (x, W, A, Bm))
    out, inn = W.shape
    r = A.shape[0]
    y = np.empty((Bt * S, out), np.float32)
    xa = np.empty((Bt * S, r), np.float32)
    lib().orc_lora_fwd(_f(x), _f(W), _f(A), _f(Bm), C.c_float(scaling), C.c_int64(Bt), C.c_int64(S), C.c_int64(inn),
                       C.c_int64(out), C.c_int64(r), _f(y), _f(xa))
    return y, xa


def lora_bwd(x, W, A, Bm, scaling, dy, Bt, S):
    """orc_lora_bwd: returns dx, dA, dB."""
    x, W, A, Bm, dy = (np.ascontiguousarray(t, np.float32) for t in (x, W, A, Bm, dy))
    out, inn = W.shape
    r = A.shape[0]
    dx = np.empty((Bt * S, inn), np.float32)
    dA = np.zeros((r, inn), np.float32)
    dB = np.zeros((out, r), np.float32)
    lib().orc_lora_bwd(_f(x), _f(W), _f(A), _f(Bm), C.c_float(scaling), _f(dy), C.c_int64(Bt), C.c_int64(S),
                       C.c_int64(inn), C.c_int64(out), C.c_int64(r), _f(dx), _f(dA), _f(dB))
    return dx, dA, dB


def lora_merge(W, A, Bm, scaling, sign=1):
    """orc_lora_merge: returns W +- (Bm A) * scaling (a new array)."""
    W = np.array(W, np.float32, copy=True, order="C")
    A, Bm = (np.ascontiguousarray(t, np.float32) for t in (A, Bm))
    out, inn = W.shape
    lib().orc_lora_merge(_f(W), _f(A), _f(Bm), C.c_float(scaling), C.c_int64(inn), C.c_int64(out),
                         C.c_int64(A.shape[0]), C.c_int(sign))
    return W


# ----------------------------------------------------------------------------- tensor primitives
DT_CODES = {np.dtype(np.float32): 0, np.dtype(np.float16): 1, np.dtype(np.int32): 3, np.dtype(np.int64): 4}
BINARY = {"add": 0, "sub": 1, "mul": 2, "div": 3}
UNARY = {"neg": 0, "abs": 1, "exp": 2, "log": 3, "sqrt": 4, "tanh": 5, "sigmoid": 6, "gelu": 7, "silu": 8}
REDUCE = {"sum": 0, "mean": 1, "max": 2, "min": 3}


def _i64arr(v):
    return np.ascontiguousarray(np.asarray(v, np.int64))


def broadcast_shape(a, b):
    out = np.zeros(max(len(a), len(b), 1), np.int64)
    r = lib().orc_broadcast_shape(_i(_i64arr(a)), C.c_int(len(a)), _i(_i64arr(b)), C.c_int(len(b)), _i(out))
    if r < 0:
        raise ValueError("shapes do not broadcast")
    return tuple(int(v) for v in out[:r])


def strided_copy(base, offset, shape, strides):
    """orc_strided_copy of the view (offset, shape, strides) (in elements) of a flat array."""
    base = np.ascontiguousarray(base)
    out = np.empty(int(np.prod(shape)) if len(shape) else 1, base.dtype)
    lib().orc_strided_copy(base.ctypes.data_as(C.c_void_p), C.c_int64(offset), C.c_int(len(shape)),
                           _i(_i64arr(shape)), _i(_i64arr(strides)), C.c_int64(base.itemsize),
                           out.ctypes.data_as(C.c_void_p))
    return out.reshape(shape)


def cast(x, to, bf16_from=False):
    """orc_cast: x (float32 / float16 / int32 / int64, or uint16 bf16 bits with bf16_from) -> `to`
    ("f32", "f16", "bf16", "i32", "i64"); 16-bit results are returned as uint16 bits."""
    x = np.ascontiguousarray(x)
    fr = 2 if bf16_from else DT_CODES[x.dtype] if x.dtype != np.uint16 else 1
    code = {"f32": 0, "f16": 1, "bf16": 2, "i32": 3, "i64": 4}[to]
    odt = {0: np.float32, 1: np.uint16, 2: np.uint16, 3: np.int32, 4: np.int64}[code]
    out = np.empty(x.shape, odt)
    rc = lib().orc_cast(x.ctypes.data_as(C.c_void_p), C.c_int(fr), out.ctypes.data_as(C.c_void_p), C.c_int(code),
                        C.c_int64(x.size))
    if rc != 0:
        raise NotImplementedError(f"cast {fr} -> {code}")
    return out


def binary(op, a, b, a_view=None, b_view=None):
    """orc_binary.  a / b are arrays (contiguous views) or flat bases with views (offset, shape, strides)."""
    def view(x, v):
        x = np.ascontiguousarray(x, np.float32)
        if v is None:
            st = [s // 4 for s in x.strides] if x.ndim else []
            return x.ravel(), 0, list(x.shape), st
        return x.ravel(), v[0], list(v[1]), list(v[2])
    xa, oa, sa, ta = view(a, a_view)
    xb, ob, sb, tb = view(b, b_view)
    shape = broadcast_shape(sa, sb)
    out = np.empty(shape, np.float32)
    rc = lib().orc_binary(C.c_int(BINARY[op]), _f(xa), C.c_int64(oa), _i(_i64arr(sa)), _i(_i64arr(ta)),
                          C.c_int(len(sa)), _f(xb), C.c_int64(ob), _i(_i64arr(sb)), _i(_i64arr(tb)), C.c_int(len(sb)),
                          _f(out))
    if rc != 0:
        raise ValueError("shapes do not broadcast")
    return out


def unary(op, x):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().orc_unary(C.c_int(UNARY[op]), _f(x), _f(y), C.c_int64(x.size))
    return y


def reduce_all(op, x):
    L = lib()
    L.orc_reduce_all.restype = C.c_float
    x = np.ascontiguousarray(x, np.float32)
    return np.float32(L.orc_reduce_all(C.c_int(REDUCE[op]), _f(x), C.c_int64(x.size)))


def reduce_dim(op, x, dim, keepdim=False):
    x = np.ascontiguousarray(x, np.float32)
    d = dim + x.ndim if dim < 0 else dim
    oshape = [s for i, s in enumerate(x.shape) if i != d]
    out = np.empty(oshape, np.float32)
    lib().orc_reduce_dim(C.c_int(REDUCE[op]), _f(x), C.c_int(x.ndim), _i(_i64arr(x.shape)), C.c_int(d), _f(out))
    if keepdim:
        out = out.reshape([1 if i == d else s for i, s in enumerate(x.shape)])
    return out


def cat(arrays, dim):
    arrays = [np.ascontiguousarray(a) for a in arrays]
    r = arrays[0].ndim
    d = dim + r if dim < 0 else dim
    outer = int(np.prod(arrays[0].shape[:d]))
    inner = int(np.prod(arrays[0].shape[d + 1:]))
    mids = _i64arr([a.shape[d] for a in arrays])
    shape = list(arrays[0].shape)
    shape[d] = int(mids.sum())
    out = np.empty(shape, arrays[0].dtype)
    ptrs = (C.c_void_p * len(arrays))(*[a.ctypes.data for a in arrays])
    lib().orc_cat(ptrs, _i(mids), C.c_int(len(arrays)), C.c_int64(outer), C.c_int64(inner),
                  C.c_int64(arrays[0].itemsize), out.ctypes.data_as(C.c_void_p))
    return out


def sum_to_shape(g, target):
    g = np.ascontiguousarray(g, np.float32)
    out = np.empty(target, np.float32)
    rc = lib().orc_sum_to_shape(_f(g), C.c_int(g.ndim), _i(_i64arr(g.shape)), C.c_int(len(target)),
                                _i(_i64arr(target)), _f(out))
    if rc != 0:
        raise ValueError("cannot reduce to the target shape")
    return out
