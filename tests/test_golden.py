"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the manifest hashes match, the oracle reproduces every stored output
bit for bit, and the stored outputs agree with an independent numpy fp64
evaluation of the same formulas (so the fixtures pin more than the oracle's
own code).  GPU: the HIP kernels reproduce the stored outputs within the
parity bar (1e-2 max-abs/relative for fp16 outputs, 1e-3 for the fp32 LSE,
identical greedy ids)."""
import os

import numpy as np
import pytest

from conftest import assert_close_f16, f32, from_dev, to_dev

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(HERE, name)) as z:  # allow_pickle stays False
        return {k: z[k] for k in z.files}


def test_manifest_hashes():
    import importlib.util
    spec = importlib.util.spec_from_file_location("make_golden", os.path.join(HERE, "make_golden.py"))
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    for line in open(os.path.join(HERE, "MANIFEST.txt")):
        digest, name = line.split()
        assert mg.content_sha256(os.path.join(HERE, name)) == digest, name


def test_oracle_reproduces_fixtures(orc):
    import importlib.util
    spec = importlib.util.spec_from_file_location("make_golden", os.path.join(HERE, "make_golden.py"))
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    for name, fn in mg.FIXTURES.items():
        fresh, stored = fn(), load(name)
        assert set(fresh) == set(stored), name
        for k in stored:
            assert np.array_equal(fresh[k], stored[k]), f"{name}:{k}"


def _f64(h):
    return f32(h).astype(np.float64)


def test_fixtures_vs_numpy_fp64():
    g = load("gemm_64.npz")
    A, B, C0 = _f64(g["a"]), _f64(g["b"]), _f64(g["c0"])
    for key, want in [("nn", A @ B), ("tn", A.T @ B), ("nt", A @ B.T), ("acc", C0 + A @ B),
                      ("bcast", _f64(g["a3"]) @ _f64(g["b3"]))]:
        assert np.abs(_f64(g[key]) - want).max() <= 1e-2 * (1 + np.abs(want).max()), key

    f = load("flash_b1h2s64.npz")
    Q, K, V = _f64(f["q"])[0].reshape(64, 2, 64), _f64(f["k"])[0], _f64(f["v"])[0]
    for causal in (0, 1):
        for h in range(2):
            s = Q[:, h] @ K.T / 8.0
            if causal:
                s[np.triu_indices(64, 1)] = -np.inf
            m = s.max(1, keepdims=True)
            p = np.exp(s - m)
            lse = (m + np.log(p.sum(1, keepdims=True)))[:, 0]
            o = (p / p.sum(1, keepdims=True)) @ V
            got = _f64(f[f"o{causal}"])[0].reshape(64, 2, 64)[:, h]
            assert np.abs(got - o).max() <= 1e-2
            assert np.abs(f[f"lse{causal}"][0, h] - lse).max() <= 1e-4

    s = load("sq_l160.npz")
    q, kc, vc = _f64(s["q"]), _f64(s["kc"]), _f64(s["vc"])
    sc = kc[:160] @ q / 8.0
    p = np.exp(sc - sc.max())
    assert np.abs(_f64(s["out"]) - (p / p.sum()) @ vc[:160]).max() <= 1e-2
    for h in range(4):
        sl = slice(16 * h, 16 * h + 16)
        sc = kc[:160, sl] @ q[sl] / 4.0
        p = np.exp(sc - sc.max())
        assert np.abs(_f64(s["out_h4"])[sl] - (p / p.sum()) @ vc[:160, sl]).max() <= 1e-2


# ----------------------------------------------------------------------------- GPU


@pytest.mark.gpu
def test_gpu_gemm_fixture(dev):
    import torch

    import evk_amd as evk
    g = load("gemm_64.npz")
    A, B = to_dev(g["a"], dev), to_dev(g["b"], dev)
    for key, ta, tb in [("nn", False, False), ("tn", True, False), ("nt", False, True)]:
        C = torch.empty((64, 64), dtype=torch.float16, device=dev)
        evk.matmul(A, B, C, ta, tb)
        torch.cuda.synchronize()
        assert_close_f16(from_dev(C), g[key], what=key)
    C = to_dev(g["c0"], dev)
    evk.matmul(A, B, C, acc_c=True)
    C3 = torch.empty((3, 64, 64), dtype=torch.float16, device=dev)
    evk.matmul(to_dev(g["a3"], dev), to_dev(g["b3"], dev), C3)
    torch.cuda.synchronize()
    assert_close_f16(from_dev(C), g["acc"], what="acc")
    assert_close_f16(from_dev(C3), g["bcast"], what="broadcast")


@pytest.mark.gpu
@pytest.mark.parametrize("causal", [0, 1])
def test_gpu_flash_fixture(dev, causal):
    import torch

    import evk_amd as evk
    f = load("flash_b1h2s64.npz")
    Q, K, V, G = (to_dev(f[k], dev) for k in ("q", "k", "v", "dO"))
    O = torch.empty_like(Q)
    L = torch.empty((1, 2, 64), dtype=torch.float32, device=dev)
    evk.flash_attention(Q, K, V, O, causal=bool(causal), lse=L)
    dQ, dK, dV = torch.empty_like(Q), torch.empty_like(K), torch.empty_like(V)
    evk.flash_attention_bwd(Q, K, V, O, G, dQ, dK, dV, causal=bool(causal), lse=L)
    torch.cuda.synchronize()
    assert_close_f16(from_dev(O), f[f"o{causal}"], what="O")
    assert np.abs(L.cpu().numpy() - f[f"lse{causal}"]).max() <= 1e-3
    for t, k in ((dQ, "dq"), (dK, "dk"), (dV, "dv")):
        assert_close_f16(from_dev(t), f[f"{k}{causal}"], what=k)


@pytest.mark.gpu
def test_gpu_sq_fixture(dev):
    import torch

    import evk_amd as evk
    s = load("sq_l160.npz")
    q, kc, vc = (to_dev(s[k], dev) for k in ("q", "kc", "vc"))
    for heads, key in ((1, "out"), (4, "out_h4")):
        out = torch.empty(64, dtype=torch.float16, device=dev)
        evk.single_query_attention(q, kc, vc, out, 160, heads)
        torch.cuda.synchronize()
        assert_close_f16(from_dev(out), s[key], what=key)


@pytest.mark.gpu
def test_gpu_decode_fixture(dev):
    import torch

    import evk_amd as evk
    import importlib.util
    spec = importlib.util.spec_from_file_location("make_golden", os.path.join(HERE, "make_golden.py"))
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    d = load("decode_d64.npz")
    cfg = evk.model_cfg(**mg.DECODE_CFG)
    W = to_dev(d["weights"], dev)
    cache = torch.zeros(evk.model_cache_elems(cfg), dtype=torch.float16, device=dev)
    prompt = torch.from_numpy(d["prompt"].view(np.int16)).to(dev)
    steps = len(d["ids"]) - 1
    tok = torch.zeros(steps + 1, dtype=torch.int16, device=dev)
    logits = torch.empty(cfg.vocab, dtype=torch.float16, device=dev)
    evk.model_prefill(cfg, W, cache, prompt, 0, tok, logits)
    evk.model_decode(cfg, W, cache, tok, steps, len(d["prompt"]), logits)
    torch.cuda.synchronize()
    assert list(from_dev(tok)) == list(d["ids"])
    assert_close_f16(from_dev(logits), d["logits"][-1], what="final logits")
