"""GPU parity of the training ops (evk_amd/csrc/train_ops.hip, through the C
ABI) against the oracle on the same seeded inputs: fp16 outputs within the
1e-2 max-abs/relative bar, exact where the op only moves, compares or adds
small integers.  Sizes cover ragged tails, misaligned views (the per-element
path of the 16-byte kernels), repeated and out-of-range ids, ignored targets
and empty tensors."""
import numpy as np
import pytest

from conftest import assert_close_f16, f32, from_dev, to_dev

pytestmark = pytest.mark.gpu


def h(x):
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def rnd(seed, shape, std=1.0):
    return h(np.random.default_rng(seed).normal(0, std, shape))


def sync():
    import torch
    torch.cuda.synchronize()


@pytest.mark.parametrize("n", [1, 7, 8, 1000, 65541])
def test_elementwise_ops(dev, orc, n):
    import evk_amd as evk
    x, g, a = rnd(n, n, 2), rnd(n + 1, n), rnd(n + 2, n)
    X, G = to_dev(x, dev), to_dev(g, dev)
    out = to_dev(np.zeros(n, np.uint16), dev)
    evk.relu(X, out)
    sync()
    assert np.array_equal(from_dev(out), orc.relu(x)), "relu"
    A = to_dev(a, dev)
    evk.relu_backward(G, X, A)
    sync()
    assert_close_f16(from_dev(A), orc.relu_backward(g, x, a), what="relu_backward")
    A = to_dev(a, dev)
    evk.gelu_backward(G, X, A)
    sync()
    assert_close_f16(from_dev(A), orc.gelu_backward(g, x, a), what="gelu_backward")
    S = to_dev(x, dev)
    evk.scale(S, -0.37)
    sync()
    assert_close_f16(from_dev(S), orc.scale(x, -0.37), what="scale")
    P = to_dev(x, dev)
    evk.sgd(P, G, 0.05)
    sync()
    assert_close_f16(from_dev(P), orc.sgd(x, g, 0.05), what="sgd")


def test_elementwise_misaligned(dev, orc):
    """Views starting 2 bytes into an allocation take the per-element path."""
    import evk_amd as evk
    n = 1003
    x, g, a = rnd(1, n + 1, 2), rnd(2, n + 1), rnd(3, n + 1)
    X, G, A = to_dev(x, dev)[1:], to_dev(g, dev)[1:], to_dev(a, dev)[1:]
    evk.gelu_backward(G, X, A)
    sync()
    assert_close_f16(from_dev(A), orc.gelu_backward(g[1:], x[1:], a[1:]), what="gelu_backward misaligned")


def test_adam_steps(dev, orc):
    import evk_amd as evk
    n = 4099
    rng = np.random.default_rng(11)
    p = h(rng.uniform(-1, 1, n))
    m = v = np.zeros(n, np.uint16)
    P, M, V = to_dev(p, dev), to_dev(m, dev), to_dev(v, dev)
    b1, b2 = 0.9, 0.999
    for t in range(1, 6):
        g = h(rng.normal(0, 0.3, n))
        g[::97] = h([np.inf])[0]  # non-finite gradients leave those elements alone
        c1, c2 = 1 / (1 - b1 ** t), 1 / (1 - b2 ** t)
        evk.adam(P, to_dev(g, dev), M, V, 1e-2, b1, b2, c1, c2, 1e-4)
        p, m, v = orc.adam(p, g, m, v, 1e-2, b1, b2, c1, c2, 1e-4)
    sync()
    assert_close_f16(from_dev(P), p, what="adam param")
    assert_close_f16(from_dev(M), m, what="adam m/rms")
    assert_close_f16(from_dev(V), v, what="adam log2 rms")


@pytest.mark.parametrize("shape,scale", [((3, 5), 1.0), ((2, 4, 129), 0.125), ((5, 1000), 1e-3), ((1, 1), 2.0),
                                         ((7, 8), 0.5), ((3, 2048), 0.25), ((2, 4096), 0.1)])
def test_softmax_and_backward(dev, orc, shape, scale):
    import evk_amd as evk
    x = rnd(21, shape, 3)
    flat = x.reshape(-1)
    flat[::7] = h([-65504])[0]  # masked entries
    X = to_dev(x, dev)
    Y = to_dev(np.zeros(shape, np.uint16), dev)
    evk.softmax(X, Y, scale)
    sync()
    p = orc.softmax(x, scale)
    assert_close_f16(from_dev(Y), p, atol=2e-3, rtol=1e-2, what="softmax")
    g, gin = rnd(22, shape), rnd(23, shape)
    GI = to_dev(gin, dev)
    evk.softmax_backward(to_dev(p, dev), to_dev(g, dev), GI, scale)
    sync()
    assert_close_f16(from_dev(GI), orc.softmax_backward(p, g, gin, scale), what="softmax_backward")


@pytest.mark.parametrize("shape", [(2, 4), (3, 7, 96), (1, 4096)])
def test_rms_norm_backward(dev, orc, shape):
    import evk_amd as evk
    x, g, a = rnd(31, shape, 2), rnd(32, shape), rnd(33, shape)
    A = to_dev(a, dev)
    evk.rms_norm_backward(to_dev(x, dev), to_dev(g, dev), A, 1e-4)
    sync()
    assert_close_f16(from_dev(A), orc.rms_norm_backward(x, g, a, 1e-4), what="rms_norm_backward")


@pytest.mark.parametrize("n", [3, 1000, 100003])
def test_mse_loss(dev, orc, n):
    import evk_amd as evk
    p, t = rnd(41, n), rnd(42, n)
    G = to_dev(np.zeros(n, np.uint16), dev)
    R = to_dev(np.zeros(1, np.uint16), dev)
    evk.mse_loss(to_dev(p, dev), to_dev(t, dev), G, R)
    sync()
    wg, wr = orc.mse_loss(p, t)
    assert_close_f16(from_dev(G), wg, what="mse grad")
    assert_close_f16(from_dev(R), wr, atol=1e-3, rtol=1e-3, what="mse loss")


@pytest.mark.parametrize("P,V", [(3, 4), (17, 1000), (64, 32000), (5, 3), (4, 32768), (3, 40000)])
def test_cross_entropy(dev, orc, P, V):
    import torch

    import evk_amd as evk
    x = rnd(51, (P, V), 3)
    rng = np.random.default_rng(52)
    t = rng.integers(0, V + 3, P).astype(np.uint16)  # includes ignored ids 0 and >= V
    t[0] = 0
    G = to_dev(np.zeros((P, V), np.uint16), dev)
    R = to_dev(np.zeros(1, np.uint16), dev)
    T = torch.from_numpy(t.view(np.int16)).to(dev)
    for _ in range(2):  # the second call reuses the library's workspace
        evk.cross_entropy_loss(to_dev(x, dev), T, G, R)
    sync()
    wg, wr = orc.cross_entropy_loss(x, t)
    assert_close_f16(from_dev(G), wg, atol=1e-3, rtol=1e-2, what="cross_entropy grad")
    assert_close_f16(from_dev(R), wr, atol=2e-3, rtol=2e-3, what="cross_entropy loss")


def test_cross_entropy_all_ignored(dev, orc):
    import torch

    import evk_amd as evk
    x = rnd(53, (4, 9))
    G = to_dev(np.ones((4, 9), np.uint16), dev)
    R = to_dev(h([5.0]), dev)
    evk.cross_entropy_loss(to_dev(x, dev), torch.zeros(4, dtype=torch.int16, device=dev), G, R)
    sync()
    assert np.all(f32(from_dev(G)) == 0) and f32(from_dev(R))[0] == 0


def test_sum_batch_mask_position(dev, orc):
    import evk_amd as evk
    x = h(np.random.default_rng(61).integers(-8, 8, (6, 1003)))
    o = h(np.full(1003, 2))
    O = to_dev(o, dev)
    evk.sum_batch(to_dev(x, dev), O, 6, 1003)
    sync()
    assert np.array_equal(from_dev(O), orc.sum_batch(x, o, 6, 1003)), "sum_batch"
    s = rnd(62, (2, 3, 37, 37))
    S = to_dev(s, dev)
    evk.apply_causal_mask(S)
    sync()
    assert np.array_equal(from_dev(S), orc.apply_causal_mask(s)), "causal mask"
    B, N, D = 3, 11, 24
    inp, pos = rnd(63, (B, N, D)), rnd(64, (N, D))
    OUT = to_dev(np.zeros((B, N, D), np.uint16), dev)
    evk.position_add(to_dev(inp, dev), to_dev(pos, dev), OUT, B, N, D)
    sync()
    assert np.array_equal(from_dev(OUT), orc.position_add(inp, pos, B, N, D)), "position_add"
    g, gi, gp = rnd(65, (B, N, D)), rnd(66, (B, N, D)), rnd(67, (N, D))
    GI, GP = to_dev(gi, dev), to_dev(gp, dev)
    evk.position_add_backward(to_dev(g, dev), GI, GP, B, N, D)
    sync()
    wi, wp = orc.position_add_backward(g, gi, gp, B, N, D)
    assert_close_f16(from_dev(GI), wi, what="position grad_in")
    assert_close_f16(from_dev(GP), wp, what="position grad_pos")


def test_rope_backward(dev, orc):
    import evk_amd as evk
    B, S, E = 2, 33, 64
    g, a = rnd(71, (B, S, E)), rnd(72, (B, S, E))
    A = to_dev(a, dev)
    evk.rope_backward(to_dev(g, dev), A, B, S, E, 10000.0)
    sync()
    assert_close_f16(from_dev(A), orc.rope_backward(g, a, B, S, E, 10000.0), what="rope_backward")


def test_embed_backward(dev, orc):
    import torch

    import evk_amd as evk
    vocab, dim, n = 50, 96, 300
    rng = np.random.default_rng(81)
    idx = rng.integers(0, vocab + 5, n).astype(np.uint16)  # repeats and ids past the table
    g, base = rnd(82, (n, dim)), rnd(83, (vocab, dim))
    GE = to_dev(base, dev)
    evk.embed_backward(to_dev(g, dev), torch.from_numpy(idx.view(np.int16)).to(dev), GE)
    sync()
    assert np.array_equal(from_dev(GE), orc.embed_backward(g, idx, base)), "embed_backward"


def test_empty_inputs(dev):
    import torch

    import evk_amd as evk
    e = torch.empty(0, dtype=torch.float16, device=dev)
    evk.relu(e, e)
    evk.scale(e, 2.0)
    evk.sgd(e, e, 0.1)
    evk.sum_batch(e, e, 3, 0)
    sync()
