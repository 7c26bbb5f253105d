"""CPU oracle for the evk AI hot path (TEST INFRASTRUCTURE ONLY).

This package wraps ``oracle/liboracle.so`` (built from ``oracle/oracle.c`` by
``oracle/Makefile``) and, when it was built, ``oracle/_ref/libevkref.so``
(the reference's own fp16 conversion and CPU matmul helpers compiled from
carloshgsilva/evk's headers).  Only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import it, and only as the
checker; the product library never calls into it.

All fp16 tensors are numpy ``uint16`` arrays holding binary16 bit patterns.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None
_REF = None

u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")


class ModelCfg(C.Structure):
    """Decode model configuration (mirrors orc_model_cfg in oracle.c)."""

    _fields_ = [
        ("vocab", C.c_uint32), ("d", C.c_uint32), ("heads", C.c_uint32),
        ("dh", C.c_uint32), ("layers", C.c_uint32), ("hidden", C.c_uint32),
        ("max_seq", C.c_uint32), ("eps", C.c_float), ("rope_base", C.c_float),
    ]


def build(force: bool = False) -> None:
    """Compile liboracle.so (and oracle/_ref when the reference is present)."""
    if force or not os.path.exists(os.path.join(_HERE, "liboracle.so")):
        subprocess.run(["make", "-s", "-C", _HERE, "all"], check=True)


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            build()
        L = C.CDLL(path)
        L.orc_f32_to_f16.restype = C.c_uint16
        L.orc_f32_to_f16.argtypes = [C.c_float]
        L.orc_f16_to_f32.restype = C.c_float
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_f16_to_f32_n.argtypes = [u16p, f32p, C.c_uint64]
        L.orc_f32_to_f16_n.argtypes = [f32p, u16p, C.c_uint64]
        L.orc_max_threads.restype = C.c_int
        L.orc_set_threads.argtypes = [C.c_int]
        L.orc_fill_uniform_f16.argtypes = [u16p, C.c_uint64, C.c_uint64, C.c_float, C.c_float]
        L.orc_fill_normal_f16.argtypes = [u16p, C.c_uint64, C.c_uint64, C.c_float, C.c_float]
        L.orc_fill_tokens_u16.argtypes = [u16p, C.c_uint64, C.c_uint64, C.c_uint32]
        mm = [u16p, u16p, u16p, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32,
              C.c_int, C.c_int, C.c_int, C.c_uint64, C.c_uint64, C.c_uint64]
        L.orc_matmul.argtypes = mm
        L.orc_matmul_naive.argtypes = mm
        L.orc_matmul_naive_rows.argtypes = [f32p, f32p, f32p, C.c_uint32, C.c_uint32,
                                            C.c_uint32, C.c_uint32]
        L.orc_attention_fwd.argtypes = [u16p, u16p, u16p, u16p, C.c_void_p, C.c_uint32,
                                        C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32,
                                        C.c_int, C.c_float]
        L.orc_attention_bwd.argtypes = [u16p, u16p, u16p, u16p, u16p, u16p, u16p,
                                        C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32,
                                        C.c_uint32, C.c_int, C.c_float]
        L.orc_sq_attention.argtypes = [u16p, u16p, u16p, u16p, C.c_uint32, C.c_uint32,
                                       C.c_uint32, C.c_uint64]
        L.orc_rms_norm.argtypes = [u16p, u16p, C.c_uint64, C.c_uint32, C.c_float]
        L.orc_rope.argtypes = [u16p, u16p, C.c_uint32, C.c_uint32, C.c_uint32, C.c_float,
                               C.c_uint32, C.c_uint32]
        L.orc_gelu_f32.restype = C.c_float
        L.orc_gelu_f32.argtypes = [C.c_float]
        L.orc_gelu.argtypes = [u16p, u16p, C.c_uint64]
        L.orc_add.argtypes = [u16p, u16p, u16p, C.c_uint64]
        L.orc_embed.argtypes = [u16p, u16p, u16p, C.c_uint64, C.c_uint32]
        L.orc_greedy_row.restype = C.c_uint16
        L.orc_greedy_row.argtypes = [u16p, C.c_uint32, C.c_uint32]
        L.orc_greedy_sample.argtypes = [u16p, u16p, C.c_uint32, C.c_uint32, C.c_uint32,
                                        C.c_uint32, C.c_uint32, C.c_uint32]
        L.orc_model_weight_elems.restype = C.c_uint64
        L.orc_model_weight_elems.argtypes = [C.POINTER(ModelCfg)]
        L.orc_model_cache_elems.restype = C.c_uint64
        L.orc_model_cache_elems.argtypes = [C.POINTER(ModelCfg)]
        L.orc_model_forward.restype = C.c_uint32
        L.orc_model_forward.argtypes = [C.POINTER(ModelCfg), u16p, u16p, u16p, C.c_uint32,
                                        C.c_uint32, u16p]
        L.orc_model_generate.argtypes = [C.POINTER(ModelCfg), u16p, u16p, u16p, C.c_uint32,
                                         C.c_uint32, u16p, C.c_void_p]
        L.orc_model_step.restype = C.c_uint32
        L.orc_model_step.argtypes = [C.POINTER(ModelCfg), u16p, u16p, C.c_uint16, C.c_uint32,
                                     u16p]
        # training ops
        L.orc_scale.argtypes = [u16p, C.c_float, C.c_uint64]
        L.orc_relu.argtypes = [u16p, u16p, C.c_uint64]
        L.orc_relu_bwd.argtypes = [u16p, u16p, u16p, C.c_uint64]
        L.orc_gelu_grad_f32.restype = C.c_float
        L.orc_gelu_grad_f32.argtypes = [C.c_float]
        L.orc_gelu_bwd.argtypes = [u16p, u16p, u16p, C.c_uint64]
        L.orc_sgd.argtypes = [u16p, u16p, C.c_float, C.c_uint64]
        L.orc_adam.argtypes = [u16p, u16p, u16p, u16p, C.c_uint64] + [C.c_float] * 6
        L.orc_softmax.argtypes = [u16p, u16p, C.c_float, C.c_uint64, C.c_uint32]
        L.orc_softmax_bwd.argtypes = [u16p, u16p, u16p, C.c_float, C.c_uint64, C.c_uint32]
        L.orc_rms_norm_bwd.argtypes = [u16p, u16p, u16p, C.c_float, C.c_uint64, C.c_uint32]
        L.orc_mse_loss.argtypes = [u16p, u16p, u16p, u16p, C.c_uint64]
        L.orc_cross_entropy.argtypes = [u16p, u16p, u16p, u16p, C.c_uint64, C.c_uint32]
        L.orc_sum_batch.argtypes = [u16p, u16p, C.c_uint32, C.c_uint64]
        L.orc_causal_mask.argtypes = [u16p, C.c_uint64, C.c_uint32]
        L.orc_position_add.argtypes = [u16p, u16p, u16p, C.c_uint32, C.c_uint64]
        L.orc_position_add_bwd.argtypes = [u16p, u16p, u16p, C.c_uint32, C.c_uint64]
        L.orc_rope_bwd.argtypes = [u16p, u16p, C.c_uint32, C.c_uint32, C.c_uint32, C.c_float]
        L.orc_embed_bwd.argtypes = [u16p, u16p, u16p, C.c_uint64, C.c_uint32, C.c_uint32]
        _LIB = L
    return _LIB


def ref():
    """The reference's own CPU helpers (oracle/_ref), or None if not built."""
    global _REF
    if _REF is None:
        path = os.path.join(_HERE, "_ref", "libevkref.so")
        if not os.path.exists(path):
            return None
        R = C.CDLL(path)
        R.ref_f32_to_f16.restype = C.c_uint16
        R.ref_f32_to_f16.argtypes = [C.c_float]
        R.ref_f16_to_f32.restype = C.c_float
        R.ref_f16_to_f32.argtypes = [C.c_uint16]
        R.ref_f16_to_f32_bits.restype = C.c_uint32
        R.ref_f16_to_f32_bits.argtypes = [C.c_uint16]
        R.ref_cpu_matmul_nn.argtypes = [f32p, f32p, f32p, C.c_uint32, C.c_uint32, C.c_uint32]
        R.ref_cpu_matmul_tn.argtypes = [f32p, f32p, f32p, C.c_uint32, C.c_uint32, C.c_uint32]
        R.ref_gelu.restype = C.c_float
        R.ref_gelu.argtypes = [C.c_float]
        _REF = R
    return _REF


# --------------------------------------------------------------------------
# numpy-level helpers
# --------------------------------------------------------------------------
def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_f16_to_f32_n(h.reshape(-1), out.reshape(-1), h.size)
    return out


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_f16_n(x.reshape(-1), out.reshape(-1), x.size)
    return out


def uniform_f16(shape, seed: int, lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
    out = np.empty(int(np.prod(shape)), np.uint16)
    lib().orc_fill_uniform_f16(out, out.size, seed, lo, hi)
    return out.reshape(shape)


def normal_f16(shape, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(int(np.prod(shape)), np.uint16)
    lib().orc_fill_normal_f16(out, out.size, seed, mean, std)
    return out.reshape(shape)


def tokens_u16(n: int, seed: int, vocab: int) -> np.ndarray:
    out = np.empty(n, np.uint16)
    lib().orc_fill_tokens_u16(out, n, seed, vocab)
    return out


def _c(x):
    return np.ascontiguousarray(x, dtype=np.uint16)


def _batch_of(shape):
    return int(np.prod(shape[:-2])) if len(shape) > 2 else 1


def matmul(a, b, c=None, transpose_a=False, transpose_b=False, acc_c=False, out_shape=None,
           naive=False):
    """C (+)= op(A).op(B) with evk::ai::matmul's batch-broadcast rules."""
    a, b = _c(a), _c(b)
    M = a.shape[-1] if transpose_a else a.shape[-2]
    K = a.shape[-2] if transpose_a else a.shape[-1]
    N = b.shape[-2] if transpose_b else b.shape[-1]
    bA, bB = _batch_of(a.shape), _batch_of(b.shape)
    if c is None:
        lead = a.shape[:-2] if bA >= bB else b.shape[:-2]
        c = np.zeros(tuple(out_shape) if out_shape else tuple(lead) + (M, N), np.uint16)
    else:
        c = np.array(c, dtype=np.uint16, copy=True, order="C")
    bC = _batch_of(c.shape)
    batch = max(bA, bB, bC)
    sA = 0 if (bA == 1 and batch > 1) else a.shape[-2] * a.shape[-1]
    sB = 0 if (bB == 1 and batch > 1) else b.shape[-2] * b.shape[-1]
    sC = c.shape[-2] * c.shape[-1]
    fn = lib().orc_matmul_naive if naive else lib().orc_matmul
    fn(a.reshape(-1), b.reshape(-1), c.reshape(-1), batch, M, N, K, int(transpose_a),
       int(transpose_b), int(acc_c), sA, sB, sC)
    return c


def attention_fwd(q, k, v, causal=False, heads_kv=1):
    """O, LSE for Q,O (B,N,H*Dh) and K,V (B,N,Hkv*Dh)."""
    q, k, v = _c(q), _c(k), _c(v)
    B, N, D = q.shape
    Dh = k.shape[2] // heads_kv
    H = D // Dh
    o = np.empty_like(q)
    lse = np.empty((B, H, N), np.float32)
    lib().orc_attention_fwd(q, k, v, o, lse.ctypes.data, B, H, heads_kv, N, Dh, int(causal),
                            float(1.0 / np.sqrt(np.float32(Dh))))
    return o, lse


def attention_bwd(q, k, v, dO, causal=False, heads_kv=1):
    q, k, v, dO = _c(q), _c(k), _c(v), _c(dO)
    B, N, D = q.shape
    Dh = k.shape[2] // heads_kv
    H = D // Dh
    dQ = np.empty_like(q)
    dK = np.empty_like(k)
    dV = np.empty_like(v)
    lib().orc_attention_bwd(q, k, v, dO, dQ, dK, dV, B, H, heads_kv, N, Dh, int(causal),
                            float(1.0 / np.sqrt(np.float32(Dh))))
    return dQ, dK, dV


def sq_attention(q, k_cache, v_cache, length, heads=1):
    q = _c(q).reshape(-1)
    kc, vc = _c(k_cache), _c(v_cache)
    row = kc.shape[-1]
    dh = q.size // heads
    out = np.empty(q.size, np.uint16)
    lib().orc_sq_attention(q, kc.reshape(-1), vc.reshape(-1), out, heads, dh, length, row)
    return out


def rms_norm(x, eps=1e-4):
    x = _c(x)
    out = np.empty_like(x)
    D = x.shape[-1]
    lib().orc_rms_norm(x.reshape(-1), out.reshape(-1), x.size // D, D, eps)
    return out


def rope(x, batch, seq, dim, base=10000.0, pos0=0, head_dim=0):
    x = _c(x)
    out = np.empty_like(x)
    lib().orc_rope(x.reshape(-1), out.reshape(-1), batch, seq, dim, base, pos0, head_dim)
    return out


def gelu(x):
    x = _c(x)
    out = np.empty_like(x)
    lib().orc_gelu(x.reshape(-1), out.reshape(-1), x.size)
    return out


def add(a, b):
    a, b = _c(a), _c(b)
    out = np.empty_like(a)
    lib().orc_add(a.reshape(-1), b.reshape(-1), out.reshape(-1), a.size)
    return out


def embed(table, idx):
    table, idx = _c(table), _c(idx)
    dim = table.shape[1]
    out = np.empty(idx.shape + (dim,), np.uint16)
    lib().orc_embed(table.reshape(-1), idx.reshape(-1), out.reshape(-1), idx.size, dim)
    return out


def greedy_sample(logits, position, token_base, token_count):
    logits = _c(logits)
    B, S, V = logits.shape
    out = np.empty(B, np.uint16)
    lib().orc_greedy_sample(logits.reshape(-1), out, B, S, V, position, token_base, token_count)
    return out


def model_cfg(vocab=32000, d=768, heads=12, layers=12, hidden=3072, max_seq=1056,
              eps=1e-4, rope_base=10000.0) -> ModelCfg:
    return ModelCfg(vocab, d, heads, d // heads, layers, hidden, max_seq, eps, rope_base)


def model_weights(cfg: ModelCfg, seed: int = 301, std: float = 0.02) -> np.ndarray:
    n = lib().orc_model_weight_elems(C.byref(cfg))
    return normal_f16((n,), seed, 0.0, std)


def model_generate(cfg: ModelCfg, weights, prompt, steps, return_logits=False):
    cache = np.zeros(lib().orc_model_cache_elems(C.byref(cfg)), np.uint16)
    ids = np.empty(steps + 1, np.uint16)
    logits = np.empty((steps + 1, cfg.vocab), np.uint16) if return_logits else None
    lib().orc_model_generate(C.byref(cfg), _c(weights), cache, _c(prompt), len(prompt), steps,
                             ids, logits.ctypes.data if logits is not None else None)
    return ids, cache, logits


def model_step(cfg: ModelCfg, weights, cache, token, pos):
    logits = np.empty(cfg.vocab, np.uint16)
    nid = lib().orc_model_step(C.byref(cfg), _c(weights), cache, int(token), int(pos), logits)
    return nid, logits


# ---------------------------------------------------------------------------
# Training ops.  fp16 arrays are uint16 bit patterns; functions that update
# in place in the reference (accumulated gradients, optimiser state) return
# updated copies here.


def scale(x, factor):
    out = _c(x).copy()
    lib().orc_scale(out.reshape(-1), factor, out.size)
    return out


def relu(x):
    x = _c(x)
    out = np.empty_like(x)
    lib().orc_relu(x.reshape(-1), out.reshape(-1), x.size)
    return out


def relu_backward(grad_out, x, grad_in):
    g, x, out = _c(grad_out), _c(x), _c(grad_in).copy()
    lib().orc_relu_bwd(g.reshape(-1), x.reshape(-1), out.reshape(-1), x.size)
    return out


def gelu_grad_f32(x):
    return lib().orc_gelu_grad_f32(float(x))


def gelu_backward(grad_out, x, grad_in):
    g, x, out = _c(grad_out), _c(x), _c(grad_in).copy()
    lib().orc_gelu_bwd(g.reshape(-1), x.reshape(-1), out.reshape(-1), x.size)
    return out


def sgd(param, grad, lr):
    out, g = _c(param).copy(), _c(grad)
    lib().orc_sgd(out.reshape(-1), g.reshape(-1), lr, out.size)
    return out


def adam(param, grad, m, v, lr, beta1, beta2, c1inv, c2inv, eps):
    """One step; returns (param, m, v) updated."""
    p, g, m, v = _c(param).copy(), _c(grad), _c(m).copy(), _c(v).copy()
    lib().orc_adam(p.reshape(-1), g.reshape(-1), m.reshape(-1), v.reshape(-1), p.size,
                   lr, beta1, beta2, c1inv, c2inv, eps)
    return p, m, v


def softmax(x, scale=1.0):
    x = _c(x)
    out = np.empty_like(x)
    D = x.shape[-1]
    lib().orc_softmax(x.reshape(-1), out.reshape(-1), scale, x.size // D, D)
    return out


def softmax_backward(probs, grad_out, grad_in, scale=1.0):
    p, g, out = _c(probs), _c(grad_out), _c(grad_in).copy()
    D = p.shape[-1]
    lib().orc_softmax_bwd(p.reshape(-1), g.reshape(-1), out.reshape(-1), scale, p.size // D, D)
    return out


def rms_norm_backward(x, grad_out, grad_in, eps=1e-4):
    x, g, out = _c(x), _c(grad_out), _c(grad_in).copy()
    D = x.shape[-1]
    lib().orc_rms_norm_bwd(x.reshape(-1), g.reshape(-1), out.reshape(-1), eps, x.size // D, D)
    return out


def mse_loss(pred, target):
    """Returns (grad, result[1])."""
    p, t = _c(pred), _c(target)
    grad = np.empty_like(p)
    res = np.zeros(1, np.uint16)
    lib().orc_mse_loss(p.reshape(-1), t.reshape(-1), grad.reshape(-1), res, p.size)
    return grad, res


def cross_entropy_loss(logits, targets):
    """logits (P, V) fp16 bits, targets (P) uint16 ids; returns (grad, result[1])."""
    x, t = _c(logits), _c(targets)
    P, V = x.shape
    grad = np.empty_like(x)
    res = np.zeros(1, np.uint16)
    lib().orc_cross_entropy(x.reshape(-1), t.reshape(-1), grad.reshape(-1), res, P, V)
    return grad, res


def sum_batch(x, out, batch, per):
    x, o = _c(x), _c(out).copy()
    lib().orc_sum_batch(x.reshape(-1), o.reshape(-1), batch, per)
    return o


def apply_causal_mask(scores):
    out = _c(scores).copy()
    N = out.shape[-1]
    lib().orc_causal_mask(out.reshape(-1), out.size // (N * N), N)
    return out


def position_add(x, pos, batch, seq, dim):
    x, pe = _c(x), _c(pos)
    out = np.empty_like(x)
    lib().orc_position_add(x.reshape(-1), pe.reshape(-1), out.reshape(-1), batch, seq * dim)
    return out


def position_add_backward(grad_out, grad_in, grad_pos, batch, seq, dim):
    g, gi, gp = _c(grad_out), _c(grad_in).copy(), _c(grad_pos).copy()
    lib().orc_position_add_bwd(g.reshape(-1), gi.reshape(-1), gp.reshape(-1), batch, seq * dim)
    return gi, gp


def rope_backward(grad_out, grad_in, batch, seq, dim, base=10000.0):
    g, out = _c(grad_out), _c(grad_in).copy()
    lib().orc_rope_bwd(g.reshape(-1), out.reshape(-1), batch, seq, dim, base)
    return out


def embed_backward(grad_out, idx, grad_emb):
    g, i, out = _c(grad_out), _c(idx), _c(grad_emb).copy()
    vocab, dim = out.shape
    lib().orc_embed_bwd(g.reshape(-1), i.reshape(-1), out.reshape(-1), i.size, dim, vocab)
    return out
