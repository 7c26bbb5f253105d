"""GPU parity: flash attention forward/backward and single-query attention
through the C ABI vs the CPU oracle (north_star bar: 1e-2 max-abs/relative,
softmax row sums within 1e-3)."""
import numpy as np
import pytest

from conftest import assert_close_f16, f32, from_dev, to_dev

pytestmark = pytest.mark.gpu


def f16(x):
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def fwd(evk, dev, q, k, v, causal):
    import torch
    Q, K, V = (to_dev(x, dev) for x in (q, k, v))
    O = torch.empty_like(Q)
    B, N, D = q.shape
    H = D // k.shape[2]
    L = torch.empty((B, H, N), dtype=torch.float32, device=dev)
    evk.flash_attention(Q, K, V, O, causal=causal, lse=L)
    torch.cuda.synchronize()
    return from_dev(O), L.cpu().numpy()


@pytest.mark.parametrize("causal", [True, False])
def test_config2_causal_flash_forward(dev, orc, causal):
    import evk_amd as evk
    B, H, S, Dh = 4, 8, 1024, 64
    q = orc.normal_f16((B, S, H * Dh), 201)
    k = orc.normal_f16((B, S, Dh), 202)
    v = orc.normal_f16((B, S, Dh), 203)
    o, lse = fwd(evk, dev, q, k, v, causal)
    wo, wl = orc.attention_fwd(q, k, v, causal)
    assert_close_f16(o, wo, what="O")
    assert np.abs(lse - wl).max() < 1e-3


@pytest.mark.parametrize("Dh", [32, 64, 128, 16, 48, 96, 256])
@pytest.mark.parametrize("N", [1, 33, 100, 130])
def test_flash_forward_ragged_heads(dev, orc, Dh, N):
    import evk_amd as evk
    B, H = 2, 3
    q = orc.normal_f16((B, N, H * Dh), 211 + N)
    k = orc.normal_f16((B, N, Dh), 212 + N)
    v = orc.normal_f16((B, N, Dh), 213 + N)
    for causal in (True, False):
        o, lse = fwd(evk, dev, q, k, v, causal)
        wo, wl = orc.attention_fwd(q, k, v, causal)
        assert_close_f16(o, wo, what=f"O Dh={Dh} N={N} causal={causal}")
        assert np.abs(lse - wl).max() < 1e-3


@pytest.mark.parametrize("order", ["growing", "shrinking"])
def test_flash_forward_moving_maximum(dev, orc, order):
    """Scores that rise (or fall) by about 18 (base 2) per 32-key chunk along
    the keys: with growing scores every chunk moves the running maximum past
    the lazy-rescale threshold, with shrinking ones most probabilities of a
    row underflow against its first chunk."""
    import evk_amd as evk
    B, H, S, Dh = 1, 8, 1024, 64
    rng = np.random.default_rng(231)
    q = f16(1.0 + 0.01 * rng.standard_normal((B, S, H * Dh)))
    ramp = np.arange(S) * 0.05 if order == "growing" else (S - 1 - np.arange(S)) * 0.05
    k = f16(ramp[None, :, None] * (1.0 + 0.01 * rng.standard_normal((B, S, Dh))))
    v = orc.normal_f16((B, S, Dh), 232)
    for causal in (True, False):
        o, lse = fwd(evk, dev, q, k, v, causal)
        wo, wl = orc.attention_fwd(q, k, v, causal)
        assert_close_f16(o, wo, what=f"O {order} causal={causal}")
        assert np.abs(lse - wl).max() < 1e-3 * max(1.0, np.abs(wl).max() / 100)


def test_flash_forward_row_sums(dev, orc):
    # V == 1 -> every output is exactly the softmax row sum: within 1e-3 of 1
    import evk_amd as evk
    B, H, S, Dh = 2, 8, 512, 64
    q = orc.normal_f16((B, S, H * Dh), 221)
    k = orc.normal_f16((B, S, Dh), 222)
    v = np.full((B, S, Dh), f16(1.0), np.uint16)
    o, lse = fwd(evk, dev, q, k, v, True)
    assert np.abs(f32(o) - 1.0).max() <= 1e-3
    # exp(s - lse) sums to one per row (fp64 from the fp16 inputs)
    Q = f32(q).astype(np.float64).reshape(B, S, H, Dh)
    K = f32(k).astype(np.float64)
    for b in range(B):
        for i in (0, 1, 255, 511):
            s = np.einsum("hd,jd->hj", Q[b, i], K[b, :i + 1]) / 8.0
            tot = np.exp(s - lse[b, :, i][:, None]).sum(1)
            assert np.abs(tot - 1).max() < 1e-3


def bwd(evk, dev, q, k, v, g, causal, use_lse):
    import torch
    Q, K, V, G = (to_dev(x, dev) for x in (q, k, v, g))
    B, N, D = q.shape
    H = D // k.shape[2]
    O = torch.empty_like(Q)
    L = torch.empty((B, H, N), dtype=torch.float32, device=dev)
    evk.flash_attention(Q, K, V, O, causal=causal, lse=L)
    dQ, dK, dV = torch.empty_like(Q), torch.empty_like(K), torch.empty_like(V)
    if use_lse:
        evk.flash_attention_bwd(Q, K, V, O, G, dQ, dK, dV, causal=causal, lse=L)
    else:
        junk = torch.full_like(Q, 7.0)  # o is not read without lse
        evk.flash_attention_bwd(Q, K, V, junk, G, dQ, dK, dV, causal=causal)
    torch.cuda.synchronize()
    return from_dev(dQ), from_dev(dK), from_dev(dV)


@pytest.mark.parametrize("use_lse", [True, False])
def test_config3_causal_flash_backward(dev, orc, use_lse):
    import evk_amd as evk
    B, H, S, Dh = 4, 8, 1024, 64
    q = orc.normal_f16((B, S, H * Dh), 201)
    k = orc.normal_f16((B, S, Dh), 202)
    v = orc.normal_f16((B, S, Dh), 203)
    g = orc.normal_f16((B, S, H * Dh), 204)
    dq, dk, dv = bwd(evk, dev, q, k, v, g, True, use_lse)
    wq, wk, wv = orc.attention_bwd(q, k, v, g, True)
    assert_close_f16(dq, wq, what="dQ")
    assert_close_f16(dk, wk, what="dK")
    assert_close_f16(dv, wv, what="dV")


@pytest.mark.parametrize("causal", [True, False])
def test_flash_backward_dh32_split_parts(dev, orc, causal):
    """Head size 32 over enough query rows (1000 positions x 4 heads) that
    the key blocks' rows are split into several parts, whose fp32 partials
    the reduce kernel sums; the last key block is ragged (1000 keys)."""
    import evk_amd as evk
    B, H, S, Dh = 2, 4, 1000, 32
    q = orc.normal_f16((B, S, H * Dh), 301)
    k = orc.normal_f16((B, S, Dh), 302)
    v = orc.normal_f16((B, S, Dh), 303)
    g = orc.normal_f16((B, S, H * Dh), 304)
    dq, dk, dv = bwd(evk, dev, q, k, v, g, causal, True)
    wq, wk, wv = orc.attention_bwd(q, k, v, g, causal)
    assert_close_f16(dq, wq, what=f"dQ dh32 causal={causal}")
    assert_close_f16(dk, wk, what=f"dK dh32 causal={causal}")
    assert_close_f16(dv, wv, what=f"dV dh32 causal={causal}")


@pytest.mark.parametrize("Dh", [32, 64, 128, 16, 48, 96, 256])
@pytest.mark.parametrize("N", [16, 45, 96])
def test_flash_backward_ragged(dev, orc, Dh, N):
    import evk_amd as evk
    B, H = 2, 2
    q = orc.normal_f16((B, N, H * Dh), 231 + N)
    k = orc.normal_f16((B, N, Dh), 232 + N)
    v = orc.normal_f16((B, N, Dh), 233 + N)
    g = orc.normal_f16((B, N, H * Dh), 234 + N)
    for causal in (True, False):
        for use_lse in (True, False):
            dq, dk, dv = bwd(evk, dev, q, k, v, g, causal, use_lse)
            wq, wk, wv = orc.attention_bwd(q, k, v, g, causal)
            tag = f"Dh={Dh} N={N} causal={causal} lse={use_lse}"
            assert_close_f16(dq, wq, what="dQ " + tag)
            assert_close_f16(dk, wk, what="dK " + tag)
            assert_close_f16(dv, wv, what="dV " + tag)


def test_flash_backward_reference_kats(dev, orc):
    # tests.h:1499-1563 (N=16, Dh=32, H=1) and tests.h:401-471 (H=2, Dh=16)
    import evk_amd as evk
    import torch
    N, Dh = 16, 32
    z = np.zeros((1, N, Dh), np.uint16)
    g = np.tile(f16(np.arange(1, Dh + 1)), (1, N, 1))
    Z = to_dev(z, dev)
    dQ, dK, dV = torch.empty_like(Z), torch.empty_like(Z), torch.empty_like(Z)
    evk.flash_attention_bwd(Z, Z, Z, Z, to_dev(g, dev), dQ, dK, dV)
    torch.cuda.synchronize()
    assert np.abs(f32(from_dev(dQ))).max() <= 5e-2 and np.abs(f32(from_dev(dK))).max() <= 5e-2
    assert np.abs(f32(from_dev(dV))[0] - np.arange(1, Dh + 1)[None, :]).max() <= 8e-2
    H, Dh = 2, 16
    q = np.zeros((1, N, H * Dh), np.uint16)
    kv = np.zeros((1, N, Dh), np.uint16)
    gg = np.zeros((1, N, H * Dh), np.uint16)
    gg[0, 0] = f16(np.arange(1, H * Dh + 1))
    Q, KV = to_dev(q, dev), to_dev(kv, dev)
    dQ, dK, dV = torch.empty_like(Q), torch.empty_like(KV), torch.empty_like(KV)
    evk.flash_attention_bwd(Q, KV, KV, Q, to_dev(gg, dev), dQ, dK, dV, heads=2)
    torch.cuda.synchronize()
    want = f32(gg)[0].reshape(N, H, Dh).sum(axis=(0, 1)) / N
    assert np.abs(f32(from_dev(dQ))).max() <= 1e-2 and np.abs(f32(from_dev(dK))).max() <= 1e-2
    assert np.abs(f32(from_dev(dV))[0] - want[None, :]).max() <= 5e-2


# ---------------------------------------------------------------------------
# single-query attention
# ---------------------------------------------------------------------------
def sq(evk, dev, q, kc, vc, L, heads):
    import torch
    Q, Kc, Vc = to_dev(q, dev), to_dev(kc, dev), to_dev(vc, dev)
    O = torch.empty_like(Q)
    evk.single_query_attention(Q, Kc, Vc, O, L, heads)
    torch.cuda.synchronize()
    return from_dev(O)


def test_sq_attention_shader_contract(dev, orc):
    # heads == 1, dim <= 64, L <= 160 (single_query_attention.comp:19-24)
    import evk_amd as evk
    for dim, L in [(64, 160), (64, 1), (32, 77), (16, 5)]:
        q = orc.normal_f16((1, 1, dim), 241 + L)
        kc = orc.normal_f16((1, 160, dim), 242 + L)
        vc = orc.normal_f16((1, 160, dim), 243 + L)
        got = sq(evk, dev, q, kc, vc, L, 1)
        assert_close_f16(got.reshape(-1), orc.sq_attention(q, kc, vc, L, 1), what=f"sq dim={dim} L={L}")


@pytest.mark.parametrize("L", [1025, 1040, 1056, 3000])
def test_sq_attention_config4(dev, orc, L):
    import evk_amd as evk
    heads, dh, maxlen = 12, 64, 3072
    q = orc.normal_f16((heads * dh,), 251 + L)
    kc = orc.normal_f16((maxlen, heads * dh), 252)
    vc = orc.normal_f16((maxlen, heads * dh), 253)
    L = min(L, maxlen)
    got = sq(evk, dev, q, kc, vc, L, heads)
    assert_close_f16(got, orc.sq_attention(q, kc, vc, L, heads), what=f"sq L={L}")
    again = sq(evk, dev, q, kc, vc, L, heads)  # split counters reset themselves
    assert np.array_equal(got, again)


def test_sq_attention_other_heads(dev, orc):
    import evk_amd as evk
    for heads, dh, L in [(4, 128, 700), (8, 16, 300), (2, 48, 90), (3, 32, 1), (1, 256, 1000), (2, 256, 65)]:
        q = orc.normal_f16((heads * dh,), 261 + dh)
        kc = orc.normal_f16((1024, heads * dh), 262)
        vc = orc.normal_f16((1024, heads * dh), 263)
        got = sq(evk, dev, q, kc, vc, L, heads)
        assert_close_f16(got, orc.sq_attention(q, kc, vc, L, heads), what=f"sq h={heads} dh={dh} L={L}")


def test_sq_attention_matches_causal_flash_row(dev, orc):
    # cross-kernel: single-query output == the last row of causal MQA flash
    import evk_amd as evk
    N, Dh = 300, 64
    q = orc.normal_f16((1, N, Dh), 271)
    k = orc.normal_f16((1, N, Dh), 272)
    v = orc.normal_f16((1, N, Dh), 273)
    o, _ = fwd(evk, dev, q, k, v, True)
    got = sq(evk, dev, q[0, N - 1], k[0], v[0], N, 1)
    assert np.abs(f32(got) - f32(o[0, N - 1])).max() <= 2e-3


def test_flash_forward_wait_timeout_is_reported(dev, orc):
    """The key-split forward's in-kernel wait is bounded: forced from the host
    to give up at once (spin limit 1, i.e. no sleep), the kernel still exits
    and raises STATUS_WAIT_TIMEOUT; with the default limit a rerun is clean
    and matches the oracle.  No wave stalls in either run."""
    import torch
    import evk_amd as evk
    B, H, S, Dh = 4, 8, 1024, 64
    q = orc.normal_f16((B, S, H * Dh), 201)
    k = orc.normal_f16((B, S, Dh), 202)
    v = orc.normal_f16((B, S, Dh), 203)
    torch.cuda.synchronize()
    evk.device_status(clear=True)
    try:
        evk.debug_set_spin_limit(1)
        for _ in range(4):
            fwd(evk, dev, q, k, v, True)
        torch.cuda.synchronize()
        forced = evk.device_status(clear=True)
    finally:
        evk.debug_set_spin_limit(0)
    assert forced & evk.STATUS_WAIT_TIMEOUT
    o, _ = fwd(evk, dev, q, k, v, True)
    torch.cuda.synchronize()
    assert evk.device_status(clear=True) == 0
    wo, _ = orc.attention_fwd(q, k, v, True)
    assert_close_f16(o, wo, what="O after the forced timeouts")


def test_flash_forward_nan_input_propagates(dev, orc):
    """A NaN in one query row makes that row's output NaN (as the reference's
    arithmetic would) and leaves every other row as the oracle has it: the
    kernels make no no-NaN assumption."""
    import evk_amd as evk
    B, H, S, Dh = 1, 2, 256, 64
    q = orc.normal_f16((B, S, H * Dh), 231)
    k = orc.normal_f16((B, S, Dh), 232)
    v = orc.normal_f16((B, S, Dh), 233)
    pos, h = 100, 1
    q[0, pos, h * Dh + 5] = 0x7E00  # fp16 quiet NaN
    for causal in (True, False):
        o, _ = fwd(evk, dev, q, k, v, causal)
        g = f32(o).reshape(B, S, H, Dh)
        assert np.isnan(g[0, pos, h]).all(), "NaN query row must give a NaN output row"
        qc = q.copy()
        qc[0, pos, h * Dh + 5] = 0
        wo, _ = orc.attention_fwd(qc, k, v, causal)
        w = f32(wo).reshape(B, S, H, Dh)
        mask = np.ones((S, H), bool)
        mask[pos, h] = False
        got, want = g[0][mask], w[0][mask]
        assert np.all(np.isfinite(got))
        assert np.abs(got - want).max() <= 1e-2 + 1e-2 * np.abs(want).max()


@pytest.mark.parametrize("B,D,heads,L", [(16, 256, 1, 160), (3, 128, 2, 700), (4, 64, 1, 33), (2, 48, 1, 90)])
def test_sq_attention_batched(dev, orc, B, D, heads, L):
    """Batched single-query attention (B sequences, each over its own cache
    (max_len, D)) against the oracle run per sequence; B=16, D=256, L=160 is
    the decode shape of example/main_llm.cpp."""
    import evk_amd as evk
    maxlen = L + 7
    q = orc.normal_f16((B, 1, D), 261 + L)
    kc = orc.normal_f16((B, maxlen, D), 262 + L)
    vc = orc.normal_f16((B, maxlen, D), 263 + L)
    got = sq(evk, dev, q, kc, vc, L, heads).reshape(B, D)
    for b in range(B):
        want = orc.sq_attention(q[b], kc[b], vc[b], L, heads)
        assert_close_f16(got[b], want, what=f"sq batched b={b}")


def test_kv_cache_write(dev, orc):
    """Rows [pos0, pos0 + n) of every sequence's cache take src; the rest of
    the cache is untouched (bit-exact), for the vector and the scalar path."""
    import torch
    import evk_amd as evk
    for D in (256, 36):
        B, S, n, pos0 = 3, 50, 7, 20
        src = orc.normal_f16((B, n, D), 271 + D)
        cache = orc.normal_f16((B, S, D), 272 + D)
        C = to_dev(cache, dev)
        evk.kv_cache_write(to_dev(src, dev), C, pos0)
        torch.cuda.synchronize()
        want = cache.copy()
        want[:, pos0:pos0 + n] = src
        assert np.array_equal(from_dev(C), want)


@pytest.mark.parametrize("D,H", [(256, 1), (96, 2)])
def test_wide_head_long_sequence(dev, orc, D, H):
    """The head-256 / head-96 MFMA kernels over a long causal sequence (1024
    positions: many key tiles per row block and many row tiles per key
    block), forward with LSE and backward, against the oracle."""
    import evk_amd as evk
    B, N = 1, 1024
    q = orc.normal_f16((B, N, H * D), 291 + D)
    k = orc.normal_f16((B, N, D), 292 + D)
    v = orc.normal_f16((B, N, D), 293 + D)
    g = orc.normal_f16((B, N, H * D), 294 + D)
    o, lse = fwd(evk, dev, q, k, v, True)
    wo, wl = orc.attention_fwd(q, k, v, True)
    assert_close_f16(o, wo, what=f"O D={D}")
    assert np.abs(lse - wl).max() < 1e-3
    dq, dk, dv = bwd(evk, dev, q, k, v, g, True, True)
    wq, wk, wv = orc.attention_bwd(q, k, v, g, True)
    assert_close_f16(dq, wq, what=f"dQ D={D}")
    assert_close_f16(dk, wk, what=f"dK D={D}")
    assert_close_f16(dv, wv, what=f"dV D={D}")


@pytest.mark.parametrize("use_lse", [True, False])
def test_reference_training_shape_d256(dev, orc, use_lse):
    """The shape the reference trains with: Graph::causal_attention over one
    head of 256 for B=16 sequences of 160 (example/main_llm.cpp:694-702,
    evk_ai.h:961-1007), forward and backward on the MFMA head-256 kernels,
    against the oracle; plus the row-sum invariant with V = 1."""
    import evk_amd as evk
    assert evk.lib().evkhip_flash_has_mfma(256) == 1
    B, N, D = 16, 160, 256
    q = orc.normal_f16((B, N, D), 281)
    k = orc.normal_f16((B, N, D), 282)
    v = orc.normal_f16((B, N, D), 283)
    g = orc.normal_f16((B, N, D), 284)
    o, lse = fwd(evk, dev, q, k, v, True)
    wo, wl = orc.attention_fwd(q, k, v, True)
    assert_close_f16(o, wo, what="O d256")
    assert np.abs(lse - wl).max() < 1e-3
    dq, dk, dv = bwd(evk, dev, q, k, v, g, True, use_lse)
    wq, wk, wv = orc.attention_bwd(q, k, v, g, True)
    assert_close_f16(dq, wq, what="dQ d256")
    assert_close_f16(dk, wk, what="dK d256")
    assert_close_f16(dv, wv, what="dV d256")
    ones = np.full((B, N, D), f16(1.0), np.uint16)
    o1, _ = fwd(evk, dev, q, k, ones, True)
    assert np.abs(f32(o1) - 1.0).max() <= 1e-3
