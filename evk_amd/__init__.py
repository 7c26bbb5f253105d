"""evk_amd - MI355X (gfx950) backend of the evk AI hot path.

Python mirror of the ``evk::ai`` operator API (reference: evk_ai.h:489-615)
over the C ABI in ``include/evkhip.h`` (``evk_amd/libevkhip.so``).  Tensors
are torch fp16 CUDA(HIP) tensors used only as device memory; every op
enqueues a hand-written gfx950 kernel on torch's current stream.  Token ids
are uint16 values stored in int16/uint16 tensors, as the reference stores
them in fp16 payload storage.

There is no CPU or PyTorch fallback: if the library is missing or a call
fails, a RuntimeError names the problem.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Optional

__all__ = [
    "lib", "available", "matmul", "flash_attention", "flash_attention_bwd",
    "single_query_attention", "rms_norm", "rope", "gelu", "add", "embed",
    "greedy_sample", "initialize", "shutdown", "ModelCfg", "model_prefill", "model_decode",
    "model_weight_elems", "model_cache_elems", "model_packed_elems", "model_pack", "model_decode_packed",
    "EvkError",
]

_HERE = os.path.dirname(os.path.abspath(__file__))
# EVKHIP_LIBRARY points the mirror at another build of the library (same ABI)
LIB_PATH = os.environ.get("EVKHIP_LIBRARY") or os.path.join(_HERE, "libevkhip.so")
_LIB = None

MAX_DIMS = 8


class EvkError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"evkhip error {code}: {msg}")
        self.code = code


class Tensor(C.Structure):
    """evkhip_tensor: device pointer + row-major shape."""

    _fields_ = [("data", C.c_void_p), ("rank", C.c_uint32), ("dims", C.c_uint32 * MAX_DIMS)]


class ModelCfg(C.Structure):
    """evkhip_model_cfg."""

    _fields_ = [
        ("vocab", C.c_uint32), ("d", C.c_uint32), ("heads", C.c_uint32), ("dh", C.c_uint32),
        ("layers", C.c_uint32), ("hidden", C.c_uint32), ("max_seq", C.c_uint32),
        ("eps", C.c_float), ("rope_base", C.c_float),
    ]


TP = C.POINTER(Tensor)

# name -> (restype, argtypes); the exports of include/evkhip.h
SIGNATURES = {
    "evkhip_version": (C.c_char_p, []),
    "evkhip_last_error": (C.c_char_p, []),
    "evkhip_init": (C.c_int, []),
    "evkhip_shutdown": (C.c_int, []),
    "evkhip_device_status": (C.c_int, [C.POINTER(C.c_uint32), C.c_int]),
    "evkhip_debug_set_spin_limit": (C.c_int, [C.c_uint32]),
    "evkhip_debug_decode_set_epoch": (C.c_int, [C.c_uint32]),
    "evkhip_debug_kv_set_launch": (C.c_int, [C.c_uint32]),
    "evkhip_flash_has_mfma": (C.c_int, [C.c_uint32]),
    "evkhip_flash_kernel_path": (C.c_int, [C.c_uint32, C.c_uint32, C.c_uint32]),
    "evkhip_kv_decode_step": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p, C.c_void_p]),
    "evkhip_matmul": (C.c_int, [TP, TP, TP, C.c_int, C.c_int, C.c_int, C.c_uint32, C.c_uint32,
                                C.c_void_p]),
    "evkhip_matmul_noalloc": (C.c_int, [TP, TP, TP, C.c_int, C.c_int, C.c_int, C.c_uint32, C.c_uint32,
                                        C.c_void_p]),
    "evkhip_flash_attention": (C.c_int, [TP, TP, TP, TP, C.c_int, C.c_void_p, C.c_void_p]),
    "evkhip_flash_attention_bwd": (C.c_int, [TP, TP, TP, TP, TP, TP, TP, TP, C.c_uint32, C.c_int,
                                             C.c_void_p, C.c_void_p]),
    "evkhip_single_query_attention": (C.c_int, [TP, TP, TP, TP, C.c_uint32, C.c_uint32, C.c_void_p]),
    "evkhip_kv_cache_write": (C.c_int, [TP, TP, C.c_uint32, C.c_void_p]),
    "evkhip_rms_norm": (C.c_int, [TP, TP, C.c_float, C.c_void_p]),
    "evkhip_rope": (C.c_int, [TP, TP, C.c_uint32, C.c_uint32, C.c_uint32, C.c_float, C.c_uint32,
                              C.c_uint32, C.c_void_p]),
    "evkhip_gelu": (C.c_int, [TP, TP, C.c_void_p]),
    "evkhip_add": (C.c_int, [TP, TP, TP, C.c_void_p]),
    "evkhip_embed": (C.c_int, [TP, TP, TP, C.c_void_p]),
    "evkhip_greedy_sample": (C.c_int, [TP, TP, C.c_uint32, C.c_uint16, C.c_uint16, C.c_void_p]),
    "evkhip_fill": (C.c_int, [C.c_void_p, C.c_uint64, C.c_uint32, C.c_void_p]),
    "evkhip_scale": (C.c_int, [TP, C.c_float, C.c_void_p]),
    "evkhip_relu": (C.c_int, [TP, TP, C.c_void_p]),
    "evkhip_relu_backward": (C.c_int, [TP, TP, TP, C.c_void_p]),
    "evkhip_gelu_backward": (C.c_int, [TP, TP, TP, C.c_void_p]),
    "evkhip_mse_loss": (C.c_int, [TP, TP, TP, TP, C.c_void_p]),
    "evkhip_sgd": (C.c_int, [TP, TP, C.c_float, C.c_void_p]),
    "evkhip_adam": (C.c_int, [TP, TP, TP, TP] + [C.c_float] * 6 + [C.c_void_p]),
    "evkhip_softmax": (C.c_int, [TP, TP, C.c_float, C.c_void_p]),
    "evkhip_softmax_backward": (C.c_int, [TP, TP, TP, C.c_float, C.c_void_p]),
    "evkhip_rms_norm_backward": (C.c_int, [TP, TP, TP, C.c_float, C.c_void_p]),
    "evkhip_cross_entropy_loss": (C.c_int, [TP, TP, TP, TP, C.c_void_p]),
    "evkhip_sum_batch": (C.c_int, [TP, TP, C.c_uint32, C.c_uint32, C.c_void_p]),
    "evkhip_apply_causal_mask": (C.c_int, [TP, C.c_void_p]),
    "evkhip_position_add": (C.c_int, [TP, TP, TP, C.c_uint32, C.c_uint32, C.c_uint32, C.c_void_p]),
    "evkhip_position_add_backward": (C.c_int, [TP, TP, TP, C.c_uint32, C.c_uint32, C.c_uint32,
                                               C.c_void_p]),
    "evkhip_rope_backward": (C.c_int, [TP, TP, C.c_uint32, C.c_uint32, C.c_uint32, C.c_float,
                                       C.c_void_p]),
    "evkhip_embed_backward": (C.c_int, [TP, TP, TP, C.c_void_p]),
    "evkhip_model_weight_elems": (C.c_uint64, [C.POINTER(ModelCfg)]),
    "evkhip_model_cache_elems": (C.c_uint64, [C.POINTER(ModelCfg)]),
    "evkhip_model_prefill": (C.c_int, [C.POINTER(ModelCfg), C.c_void_p, C.c_void_p, C.c_void_p,
                                       C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p]),
    "evkhip_model_decode": (C.c_int, [C.POINTER(ModelCfg), C.c_void_p, C.c_void_p, C.c_void_p,
                                      C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p]),
    "evkhip_model_packed_elems": (C.c_uint64, [C.POINTER(ModelCfg)]),
    "evkhip_model_pack": (C.c_int, [C.POINTER(ModelCfg), C.c_void_p, C.c_void_p, C.c_void_p]),
    "evkhip_model_decode_packed": (C.c_int, [C.POINTER(ModelCfg), C.c_void_p, C.c_void_p, C.c_void_p,
                                             C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p]),
}


def lib():
    """Load libevkhip.so (raises if it was not built)."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run `python -m evk_amd.build` "
                               "(the HIP kernels have no fallback)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def available() -> bool:
    return os.path.exists(LIB_PATH)


def _check(rc: int) -> None:
    if rc != 0:
        raise EvkError(rc, lib().evkhip_last_error().decode())


def desc(t, shape=None) -> Tensor:
    """Descriptor of a contiguous torch tensor (or a (ptr, shape) pair)."""
    if isinstance(t, tuple):
        ptr, shape = t
    else:
        if not t.is_contiguous():
            raise ValueError("evk_amd ops take contiguous tensors")
        ptr = t.data_ptr()
        shape = tuple(t.shape) if shape is None else tuple(shape)
    if len(shape) > MAX_DIMS:
        raise ValueError("rank > 8")
    d = Tensor()
    d.data = ptr
    d.rank = len(shape)
    for i, s in enumerate(shape):
        d.dims[i] = int(s)
    return d


def _stream(stream=None):
    if stream is not None:
        return C.c_void_p(int(stream))
    import torch
    if torch.cuda.is_available():
        return C.c_void_p(torch.cuda.current_stream().cuda_stream)
    return C.c_void_p(0)


def _ref(d: Tensor):
    return C.byref(d)


# ---------------------------------------------------------------------------
# evk::ai ops
# ---------------------------------------------------------------------------
def initialize() -> None:
    """evk::ai::initialize (evk_ai.cpp:211-246)."""
    _check(lib().evkhip_init())


def shutdown() -> None:
    """evk::ai::shutdown (evk_ai.cpp:248-252): frees library workspace."""
    _check(lib().evkhip_shutdown())


STATUS_WAIT_TIMEOUT = 1


def device_status(clear=False) -> int:
    """Device status bits (STATUS_*) raised by the kernels; synchronise first."""
    v = C.c_uint32(0)
    _check(lib().evkhip_device_status(C.byref(v), int(bool(clear))))
    return v.value


def debug_decode_set_epoch(distance: int) -> None:
    """Test hook: the persistent decode's hand-over tags `distance` below the
    point where they wrap (the next launch needing more clears and restarts)."""
    _check(lib().evkhip_debug_decode_set_epoch(int(distance)))


def debug_kv_set_launch(distance: int) -> None:
    """Test hook: the fused KV decode step's launch counter `distance` launches
    below the point where its hand-over tags wrap."""
    _check(lib().evkhip_debug_kv_set_launch(int(distance)))


def debug_set_spin_limit(iterations: int) -> None:
    """Test hook: iterations of the bounded in-kernel waits (0 = default)."""
    _check(lib().evkhip_debug_set_spin_limit(int(iterations)))


def matmul(a, b, c, transpose_a=False, transpose_b=False, acc_c=False, TILE_M=80, TILE_N=80,
           stream=None):
    """evk::ai::matmul (evk_ai.h:495): C (+)= op(A) . op(B) with batch broadcast."""
    da, db, dc = desc(a), desc(b), desc(c)
    _check(lib().evkhip_matmul(_ref(da), _ref(db), _ref(dc), int(transpose_a), int(transpose_b),
                               int(acc_c), int(TILE_M), int(TILE_N), _stream(stream)))
    return c


def flash_attention(q, k, v, o, causal=False, lse=None, stream=None):
    """evk::ai::flash_attention (evk_ai.h:501) + causal/LSE extensions.

    q, o: (B, N, H*Dh) fp16; k, v: (B, N, Dh) fp16; lse: optional (B, H, N) fp32.
    """
    dq, dk, dv, do = desc(q), desc(k), desc(v), desc(o)
    lp = None
    if lse is not None:
        if not lse.is_contiguous():
            raise ValueError("lse must be contiguous")
        lp = C.c_void_p(lse.data_ptr())
    _check(lib().evkhip_flash_attention(_ref(dq), _ref(dk), _ref(dv), _ref(do), int(causal), lp,
                                        _stream(stream)))
    return o


def flash_attention_bwd(q, k, v, o, dO, dQ, dK, dV, heads=0, causal=False, lse=None, stream=None):
    """evk::ai::flash_attention_bwd (evk_ai.h:503) + causal/LSE extensions."""
    ds = [desc(t) for t in (q, k, v, o, dO, dQ, dK, dV)]
    lp = C.c_void_p(lse.data_ptr()) if lse is not None else None
    _check(lib().evkhip_flash_attention_bwd(*[_ref(d) for d in ds], int(heads), int(causal), lp,
                                            _stream(stream)))


def single_query_attention(q, k_cache, v_cache, out, current_length, heads=1, stream=None):
    """Decode-step attention (single_query_attention.comp, generalised)."""
    _check(lib().evkhip_single_query_attention(_ref(desc(q)), _ref(desc(k_cache)),
                                               _ref(desc(v_cache)), _ref(desc(out)),
                                               int(current_length), int(heads), _stream(stream)))
    return out


def kv_cache_write(src, cache, pos0, stream=None):
    """Rows [pos0, pos0+n) of each sequence's cache (B, max_seq, D) <- src (B, n, D)."""
    _check(lib().evkhip_kv_cache_write(_ref(desc(src)), _ref(desc(cache)), int(pos0), _stream(stream)))


def rms_norm(inp, out, eps=1e-4, stream=None):
    _check(lib().evkhip_rms_norm(_ref(desc(inp)), _ref(desc(out)), float(eps), _stream(stream)))
    return out


def rope(inp, out, batch_size, seq_len, embed_dim, rotary_base=10000.0, position_offset=0,
         head_dim=0, stream=None):
    _check(lib().evkhip_rope(_ref(desc(inp)), _ref(desc(out)), int(batch_size), int(seq_len),
                             int(embed_dim), float(rotary_base), int(position_offset),
                             int(head_dim), _stream(stream)))
    return out


def gelu(inp, out, stream=None):
    _check(lib().evkhip_gelu(_ref(desc(inp)), _ref(desc(out)), _stream(stream)))
    return out


def add(a, b, c, stream=None):
    _check(lib().evkhip_add(_ref(desc(a)), _ref(desc(b)), _ref(desc(c)), _stream(stream)))
    return c


def embed(embeddings, indices, out, stream=None):
    _check(lib().evkhip_embed(_ref(desc(embeddings)), _ref(desc(indices)), _ref(desc(out)),
                              _stream(stream)))
    return out


# ---- training ops (evk_ai.h:507-614); *_backward accumulate into grad_in ----

def _D(t):
    return _ref(desc(t))


def scale(t, factor, stream=None):
    _check(lib().evkhip_scale(_D(t), float(factor), _stream(stream)))
    return t


def relu(inp, out, stream=None):
    _check(lib().evkhip_relu(_D(inp), _D(out), _stream(stream)))
    return out


def relu_backward(grad_out, inp, grad_in, stream=None):
    _check(lib().evkhip_relu_backward(_D(grad_out), _D(inp), _D(grad_in), _stream(stream)))
    return grad_in


def gelu_backward(grad_out, inp, grad_in, stream=None):
    _check(lib().evkhip_gelu_backward(_D(grad_out), _D(inp), _D(grad_in), _stream(stream)))
    return grad_in


def mse_loss(predicted, target, pred_grad, result, stream=None):
    _check(lib().evkhip_mse_loss(_D(predicted), _D(target), _D(pred_grad), _D(result), _stream(stream)))
    return result


def sgd(param, gradient, learning_rate, stream=None):
    _check(lib().evkhip_sgd(_D(param), _D(gradient), float(learning_rate), _stream(stream)))
    return param


def adam(param, gradient, m_state, v_state, learning_rate, beta1, beta2, beta1_correction_inv,
         beta2_correction_inv, epsilon, stream=None):
    _check(lib().evkhip_adam(_D(param), _D(gradient), _D(m_state), _D(v_state), float(learning_rate),
                             float(beta1), float(beta2), float(beta1_correction_inv),
                             float(beta2_correction_inv), float(epsilon), _stream(stream)))
    return param


def softmax(inp, out, input_scale=1.0, stream=None):
    _check(lib().evkhip_softmax(_D(inp), _D(out), float(input_scale), _stream(stream)))
    return out


def softmax_backward(probs, grad_out, grad_in, scale=1.0, stream=None):
    _check(lib().evkhip_softmax_backward(_D(probs), _D(grad_out), _D(grad_in), float(scale),
                                         _stream(stream)))
    return grad_in


def rms_norm_backward(inp, grad_out, grad_in, eps=1e-4, stream=None):
    _check(lib().evkhip_rms_norm_backward(_D(inp), _D(grad_out), _D(grad_in), float(eps), _stream(stream)))
    return grad_in


def cross_entropy_loss(logits, targets, grad, result, stream=None):
    _check(lib().evkhip_cross_entropy_loss(_D(logits), _D(targets), _D(grad), _D(result), _stream(stream)))
    return result


def sum_batch(inp, out, batch_count, size_per_batch, stream=None):
    _check(lib().evkhip_sum_batch(_D(inp), _D(out), int(batch_count), int(size_per_batch), _stream(stream)))
    return out


def apply_causal_mask(scores, stream=None):
    _check(lib().evkhip_apply_causal_mask(_D(scores), _stream(stream)))
    return scores


def position_add(inp, pos_emb, out, batch_size, seq_len, embed_dim, stream=None):
    _check(lib().evkhip_position_add(_D(inp), _D(pos_emb), _D(out), int(batch_size), int(seq_len),
                                     int(embed_dim), _stream(stream)))
    return out


def position_add_backward(grad_out, grad_in, grad_pos, batch_size, seq_len, embed_dim, stream=None):
    _check(lib().evkhip_position_add_backward(_D(grad_out), _D(grad_in), _D(grad_pos), int(batch_size),
                                              int(seq_len), int(embed_dim), _stream(stream)))
    return grad_in, grad_pos


def rope_backward(grad_out, grad_in, batch_size, seq_len, embed_dim, rotary_base=10000.0, stream=None):
    _check(lib().evkhip_rope_backward(_D(grad_out), _D(grad_in), int(batch_size), int(seq_len),
                                      int(embed_dim), float(rotary_base), _stream(stream)))
    return grad_in


def embed_backward(grad_out, indices, grad_embeddings, stream=None):
    _check(lib().evkhip_embed_backward(_D(grad_out), _D(indices), _D(grad_embeddings), _stream(stream)))
    return grad_embeddings


def greedy_sample(logits, out_tokens, position, token_base, token_count, stream=None):
    _check(lib().evkhip_greedy_sample(_ref(desc(logits)), _ref(desc(out_tokens)), int(position),
                                      int(token_base), int(token_count), _stream(stream)))
    return out_tokens


# ---------------------------------------------------------------------------
# KV-cached decode model
# ---------------------------------------------------------------------------
def model_cfg(vocab=32000, d=768, heads=12, layers=12, hidden=3072, max_seq=1056, eps=1e-4,
              rope_base=10000.0) -> ModelCfg:
    return ModelCfg(vocab, d, heads, d // heads, layers, hidden, max_seq, eps, rope_base)


def model_weight_elems(cfg: ModelCfg) -> int:
    return int(lib().evkhip_model_weight_elems(C.byref(cfg)))


def model_cache_elems(cfg: ModelCfg) -> int:
    return int(lib().evkhip_model_cache_elems(C.byref(cfg)))


def model_prefill(cfg: ModelCfg, weights, cache, tokens, pos0, next_id, logits, stream=None):
    """Runs the prompt `tokens` (int16 device tensor) from position pos0;
    next_id[0] receives the greedy id after the last prompt token."""
    _check(lib().evkhip_model_prefill(C.byref(cfg), C.c_void_p(weights.data_ptr()),
                                      C.c_void_p(cache.data_ptr()), C.c_void_p(tokens.data_ptr()),
                                      int(tokens.numel()), int(pos0), C.c_void_p(next_id.data_ptr()),
                                      C.c_void_p(logits.data_ptr()), _stream(stream)))


def model_decode(cfg: ModelCfg, weights, cache, token_io, n_steps, pos0, logits, stream=None):
    """n_steps greedy steps: token_io[s] in, token_io[s+1] out."""
    if token_io.numel() < n_steps + 1:
        raise ValueError("token_io needs n_steps+1 entries")
    _check(lib().evkhip_model_decode(C.byref(cfg), C.c_void_p(weights.data_ptr()),
                                     C.c_void_p(cache.data_ptr()), C.c_void_p(token_io.data_ptr()),
                                     int(n_steps), int(pos0), C.c_void_p(logits.data_ptr()),
                                     _stream(stream)))


def model_packed_elems(cfg: ModelCfg) -> int:
    return int(lib().evkhip_model_packed_elems(C.byref(cfg)))


def model_pack(cfg: ModelCfg, weights, packed, stream=None):
    """Writes the persistent decode's layout of `weights` into `packed`
    (model_packed_elems(cfg) fp16 elements)."""
    if packed.numel() < model_packed_elems(cfg):
        raise ValueError("packed needs model_packed_elems(cfg) elements")
    _check(lib().evkhip_model_pack(C.byref(cfg), C.c_void_p(weights.data_ptr()), C.c_void_p(packed.data_ptr()),
                                   _stream(stream)))


def model_decode_packed(cfg: ModelCfg, packed, cache, token_io, n_steps, pos0, logits, stream=None):
    """model_decode over packed weights, every step in one persistent launch."""
    if token_io.numel() < n_steps + 1:
        raise ValueError("token_io needs n_steps+1 entries")
    _check(lib().evkhip_model_decode_packed(C.byref(cfg), C.c_void_p(packed.data_ptr()),
                                            C.c_void_p(cache.data_ptr()), C.c_void_p(token_io.data_ptr()),
                                            int(n_steps), int(pos0), C.c_void_p(logits.data_ptr()),
                                            _stream(stream)))
