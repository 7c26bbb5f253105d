"""Writes the golden fixtures of this directory from the CPU oracle.

    python tests/golden/make_golden.py

Each fixture is an .npz of fp16 bit patterns (uint16), fp32 LSE rows and
uint16 token ids -- inputs and expected outputs -- generated from the seeds
below with the oracle's portable PRNG; MANIFEST.txt lists a SHA-256 of
each file's arrays (content_sha256).  The oracle is pinned to the reference elsewhere (known answers
of example/tests.h, closed forms, the compiled reference float16_t and CPU
GEMM); these fixtures freeze its outputs so any later change to the oracle
or to a kernel is caught against the same vectors.

Fixtures (shapes from the reference's own small cases):
  gemm_64.npz         64x64x64 NN, TN, NT, acc (C += A.B), broadcast A over batch 3
  flash_b1h2s64.npz   MQA flash forward/backward, B=1 H=2 S=64 Dh=64, causal and
                      not, with the fp32 row LSE
  sq_l160.npz         single-query attention, L=160 (of 192 cache rows), dim 64, 1 head;
                      and 4 heads x 16
  decode_d64.npz      2-layer decode model d=64 (2 heads x 32, hidden 128,
                      vocab 512): 6-token prompt, 5 greedy steps, final logits
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle as orc  # noqa: E402

DECODE_CFG = dict(vocab=512, d=64, heads=2, layers=2, hidden=128, max_seq=16)


def gemm():
    out = {}
    a = orc.uniform_f16((64, 64), 601)
    b = orc.uniform_f16((64, 64), 602)
    c0 = orc.uniform_f16((64, 64), 603)
    out["a"], out["b"], out["c0"] = a, b, c0
    out["nn"] = orc.matmul(a, b)
    out["tn"] = orc.matmul(a, b, transpose_a=True)
    out["nt"] = orc.matmul(a, b, transpose_b=True)
    out["acc"] = orc.matmul(a, b, c=c0, acc_c=True)
    a3 = orc.uniform_f16((1, 64, 64), 604)
    b3 = orc.uniform_f16((3, 64, 64), 605)
    out["a3"], out["b3"] = a3, b3
    out["bcast"] = orc.matmul(a3, b3, out_shape=(3, 64, 64))
    return out


def flash():
    out = {}
    B, H, S, Dh = 1, 2, 64, 64
    q = orc.normal_f16((B, S, H * Dh), 611)
    k = orc.normal_f16((B, S, Dh), 612)
    v = orc.normal_f16((B, S, Dh), 613)
    g = orc.normal_f16((B, S, H * Dh), 614)
    out.update(q=q, k=k, v=v, dO=g)
    for causal in (0, 1):
        o, lse = orc.attention_fwd(q, k, v, bool(causal))
        dq, dk, dv = orc.attention_bwd(q, k, v, g, bool(causal))
        out.update({f"o{causal}": o, f"lse{causal}": lse.astype(np.float32),
                    f"dq{causal}": dq, f"dk{causal}": dk, f"dv{causal}": dv})
    return out


def sq():
    out = {}
    q = orc.normal_f16((64,), 621)
    kc = orc.normal_f16((192, 64), 622)
    vc = orc.normal_f16((192, 64), 623)
    out.update(q=q, kc=kc, vc=vc, out=orc.sq_attention(q, kc, vc, 160, 1))
    out["out_h4"] = orc.sq_attention(q, kc, vc, 160, 4)
    return out


def decode():
    cfg = orc.model_cfg(**DECODE_CFG)
    w = orc.model_weights(cfg, seed=631, std=0.1)
    prompt = orc.tokens_u16(6, 632, DECODE_CFG["vocab"])
    ids, _, logits = orc.model_generate(cfg, w, prompt, 5, return_logits=True)
    return {"weights": w, "prompt": prompt, "ids": np.asarray(ids, np.uint16),
            "logits": np.asarray(logits, np.uint16)}


FIXTURES = {"gemm_64.npz": gemm, "flash_b1h2s64.npz": flash, "sq_l160.npz": sq, "decode_d64.npz": decode}


def content_sha256(path):
    """SHA-256 over every array's name, dtype, shape and bytes, in name order
    (independent of the zip container's own metadata)."""
    h = hashlib.sha256()
    with np.load(path) as z:
        for k in sorted(z.files):
            a = z[k]
            h.update(f"{k}:{a.dtype.str}:{a.shape};".encode())
            h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def main():
    orc.build()
    lines = []
    for name, fn in FIXTURES.items():
        arrays = fn()
        path = os.path.join(HERE, name)
        np.savez_compressed(path, **arrays)
        lines.append(f"{content_sha256(path)}  {name}")
        print("wrote", name, {k: v.shape for k, v in arrays.items()})
    open(os.path.join(HERE, "MANIFEST.txt"), "w").write("\n".join(lines) + "\n")


if __name__ == "__main__":
    main()
