"""CPU pins of the oracle's training ops (oracle/oracle.c orc_scale ..
orc_embed_bwd).  Each function is checked against the reference's own known
answers (example/tests.h) and against what the mathematics fixes, computed
here independently in fp64 numpy (finite differences, adjoint identities,
closed forms), so that a dropped term, a wrong sign or a transposed index in
the oracle fails."""
import numpy as np
import pytest

from conftest import f32


def h(x):
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def rng(seed):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------- reference KATs


def test_mse_loss_kat(orc):  # tests.h:221-263
    grad, res = orc.mse_loss(h([1, 2, 3]), h([1, 2, 4]))
    assert abs(f32(res)[0] - 1 / 3) < 1e-3
    assert np.allclose(f32(grad), [0, 0, -2 / 3], atol=5e-3)


def test_cross_entropy_kat(orc):  # tests.h:265-399
    logits = h([[0, 0, 0, 0], [0, 0, 2, 0], [1, -1, 0.5, 0]])
    targets = np.array([1, 3, 0], np.uint16)
    grad, res = orc.cross_entropy_loss(logits, targets)
    x = f32(logits).astype(np.float64)
    want_g = np.zeros_like(x)
    total = 0.0
    for r in range(2):
        p = np.exp(x[r] - x[r].max())
        p /= p.sum()
        want_g[r] = p
        want_g[r, targets[r]] -= 1
        total += -np.log(p[targets[r]])
    want_g /= 2
    assert abs(f32(res)[0] - total / 2) < 5e-3
    assert np.abs(f32(grad) - want_g).max() < 1e-2
    assert np.all(f32(grad)[2] == 0)  # ignored row
    # every position ignored: zero loss, zero gradients
    g2, r2 = orc.cross_entropy_loss(h(0.1 * np.arange(6).reshape(2, 3)), np.zeros(2, np.uint16))
    assert f32(r2)[0] == 0 and np.all(f32(g2) == 0)


def test_softmax_kat(orc):  # tests.h:619-679
    x = np.tile(np.arange(5, dtype=np.float32) - 2, (6, 1)).reshape(2, 3, 5)
    p = f32(orc.softmax(h(x)))
    assert np.abs(p.sum(-1) - 1).max() < 5e-3
    m = f32(orc.softmax(h([[0, -65504, 1, -65504]]), 1e-5))[0]
    assert m[1] == 0 and m[3] == 0 and abs(m[0] + m[2] - 1) < 5e-3 and m[0] > 0.49 and m[2] > 0.49


def test_sgd_relu_scale_kats(orc):  # tests.h:1109-1167, 1199-1222
    p = f32(orc.sgd(h([1, -2, 0.5, 4]), h([0.5, -1, 2, 0]), 0.1))
    assert np.allclose(p, [0.95, -1.9, 0.3, 4.0], atol=2e-2)
    x = h([-2, 0, 1.5, 3])
    assert np.allclose(f32(orc.relu(x)), [0, 0, 1.5, 3])
    g = orc.relu_backward(h([1, 1, 1, 1]), x, h([0, 0, 0, 0]))
    assert np.allclose(f32(g), [0, 0, 1, 1])
    assert np.allclose(f32(orc.scale(h([2, -4, 1, 0.5]), 0.5)), [1, -2, 0.5, 0.25])


def test_embed_backward_kat(orc):  # tests.h:1224-1272
    gout = h(np.arange(1, 7).reshape(2, 3))
    g = f32(orc.embed_backward(gout, np.array([1, 3], np.uint16), h(np.zeros((4, 3)))))
    want = np.zeros((4, 3))
    want[1] = [1, 2, 3]
    want[3] = [4, 5, 6]
    assert np.array_equal(g, want)


def test_position_add_kat(orc):  # tests.h:1274-1316
    pos = h(np.arange(1, 7).reshape(2, 3))
    out = f32(orc.position_add(h(np.zeros((2, 2, 3))), pos, 2, 2, 3))
    assert np.array_equal(out, np.stack([f32(pos)] * 2))
    gi, gp = orc.position_add_backward(h(np.ones((2, 2, 3))), h(np.zeros((2, 2, 3))), h(np.zeros((2, 3))), 2, 2, 3)
    assert np.all(f32(gi) == 1) and np.all(f32(gp) == 2)


def test_rope_backward_kat(orc):  # tests.h:1318-1385
    g = np.array([1, 0, 1, 0, 0, 1, 0, 1], np.float32).reshape(1, 2, 4)
    got = f32(orc.rope_backward(h(g), h(np.zeros_like(g)), 1, 2, 4))
    for t in range(2):
        for pair in range(2):
            i = t * 4 + 2 * pair
            a = t * 10000.0 ** (-2 * pair / 4)
            c, s = np.cos(a), np.sin(a)
            g0, g1 = g.reshape(-1)[i], g.reshape(-1)[i + 1]
            assert abs(got.reshape(-1)[i] - (g0 * c + g1 * s)) < 3e-2
            assert abs(got.reshape(-1)[i + 1] - (-g0 * s + g1 * c)) < 3e-2


def test_sum_batch_kat(orc):  # tests.h:1387-1409
    out = f32(orc.sum_batch(h([[1, 2, 3], [4, 5, 6]]), h([1, 1, 1]), 2, 3))
    assert np.array_equal(out, [6, 8, 10])


def test_rms_norm_backward_kat(orc):  # tests.h:1411-1470
    x = np.array([[3, 4, 0, 0], [1, 2, 3, 4]], np.float32)
    g = f32(orc.rms_norm_backward(h(x), h(np.ones_like(x)), h(np.zeros_like(x))))
    for r in range(2):
        rms = np.sqrt((x[r] ** 2).mean() + 1e-4)
        dot = (x[r] / rms).sum()
        want = 1 / rms - x[r] / rms ** 2 * dot / 4
        assert np.abs(g[r] - want).max() < 4e-2


def test_adam_kat(orc):  # tests.h:681-730: ten steps move every parameter against its gradient
    p, g = h([1, 2, 3, 4]), h([0.1, 0.2, 0.3, 0.4])
    m = v = np.zeros(4, np.uint16)
    for t in range(1, 11):
        p, m, v = orc.adam(p, g, m, v, 0.1, 0.9, 0.999, 1 / (1 - 0.9 ** t), 1 / (1 - 0.999 ** t), 1e-4)
    assert np.all(f32(p) < np.array([1, 2, 3, 4]))


# ------------------------------------------------------- mathematics (fp64 numpy)


def test_adam_tracks_fp32_adam(orc):
    """The fp16 (m / rms, log2 rms) state tracks plain fp64 Adam (cf.
    tests.h:732-844, the reference's own fp16-vs-fp32 check)."""
    r = rng(1)
    n, lr, b1, b2, eps = 64, 1e-2, 0.9, 0.999, 1e-4
    p = r.uniform(-1, 1, n).astype(np.float32)
    ph, mh, vh = h(p), np.zeros(n, np.uint16), np.zeros(n, np.uint16)
    pd, md, vd = f32(ph).astype(np.float64), np.zeros(n), np.zeros(n)
    for t in range(1, 21):
        g = h(r.normal(0, 0.5, n))
        ph, mh, vh = orc.adam(ph, g, mh, vh, lr, b1, b2, 1 / (1 - b1 ** t), 1 / (1 - b2 ** t), eps)
        gd = f32(g).astype(np.float64)
        md = b1 * md + (1 - b1) * gd
        vd = b2 * vd + (1 - b2) * gd * gd
        pd -= lr * (md / (1 - b1 ** t)) / (np.sqrt(vd / (1 - b2 ** t)) + eps)
    assert np.abs(f32(ph) - pd).max() < 3e-2
    # a non-finite gradient leaves parameter and state unchanged
    bad = h([np.inf] * n)
    p2, m2, v2 = orc.adam(ph, bad, mh, vh, lr, b1, b2, 1.0, 1.0, eps)
    assert np.array_equal(p2, ph) and np.array_equal(m2, mh) and np.array_equal(v2, vh)


def test_gelu_grad_is_the_derivative(orc):
    xs = np.linspace(-6, 6, 241)
    e = 1e-3
    for x in xs:
        num = (orc.lib().orc_gelu_f32(float(x + e)) - orc.lib().orc_gelu_f32(float(x - e))) / (2 * e)
        assert abs(orc.gelu_grad_f32(x) - num) < 2e-3, x
    x = h(rng(2).normal(0, 2, 512))
    gout = h(rng(3).normal(0, 1, 512))
    gin = h(rng(4).normal(0, 1, 512))
    got = f32(orc.gelu_backward(gout, x, gin))
    want = f32(gin) + f32(gout) * np.array([orc.gelu_grad_f32(v) for v in f32(x)])
    assert np.abs(got - want).max() <= 2e-3 * (1 + np.abs(want).max())


def test_softmax_and_backward_math(orc):
    r = rng(5)
    x = h(r.normal(0, 2, (7, 33)))
    sc = 0.37
    p = f32(orc.softmax(x, sc)).astype(np.float64)
    xd = f32(x).astype(np.float64) * sc
    want = np.exp(xd - xd.max(-1, keepdims=True))
    want /= want.sum(-1, keepdims=True)
    assert np.abs(p - want).max() < 1e-3
    # backward: grad_in += J^T g with J = (diag(p) - p p^T) * scale, rows independent
    ph = orc.softmax(x, sc)
    g = h(r.normal(0, 1, (7, 33)))
    gin = h(r.normal(0, 1, (7, 33)))
    got = f32(orc.softmax_backward(ph, g, gin, sc)).astype(np.float64)
    pp, gg = f32(ph).astype(np.float64), f32(g).astype(np.float64)
    for i in range(7):
        J = (np.diag(pp[i]) - np.outer(pp[i], pp[i])) * sc
        assert np.abs(got[i] - (f32(gin)[i] + J.T @ gg[i])).max() < 2e-2


def test_rms_norm_backward_finite_differences(orc):
    r = rng(6)
    D, eps = 24, 1e-4
    x = f32(h(r.normal(0, 1.5, (3, D)))).astype(np.float64)
    g = f32(h(r.normal(0, 1, (3, D)))).astype(np.float64)
    got = f32(orc.rms_norm_backward(h(x), h(g), h(np.zeros_like(x)), eps))

    def loss(row, v):
        return (g[row] * v / np.sqrt((v ** 2).mean() + eps)).sum()

    for row in range(3):
        num = np.zeros(D)
        for j in range(D):
            e = np.zeros(D)
            e[j] = 1e-5
            num[j] = (loss(row, x[row] + e) - loss(row, x[row] - e)) / 2e-5
        assert np.abs(got[row] - num).max() < 1e-2 * (1 + np.abs(num).max())


def test_rope_backward_is_the_adjoint(orc):
    """<rope(x), g> == <x, rope_backward(g)> with rope applied in fp64 here."""
    r = rng(7)
    B, S, E = 2, 5, 8
    x = r.normal(0, 1, (B, S, E))
    g = f32(h(r.normal(0, 1, (B, S, E)))).astype(np.float64)
    y = np.empty_like(x)
    for t in range(S):
        for p in range(E // 2):
            a = t * 10000.0 ** (-2 * p / E)
            c, s = np.cos(a), np.sin(a)
            y[:, t, 2 * p] = x[:, t, 2 * p] * c - x[:, t, 2 * p + 1] * s
            y[:, t, 2 * p + 1] = x[:, t, 2 * p] * s + x[:, t, 2 * p + 1] * c
    bt = f32(orc.rope_backward(h(g), h(np.zeros_like(g)), B, S, E)).astype(np.float64)
    assert abs((y * g).sum() - (x * bt).sum()) < 1e-2 * np.abs(x * bt).sum() / np.sqrt(x.size)


def test_cross_entropy_random(orc):
    r = rng(8)
    P, V = 9, 50
    x = h(r.normal(0, 3, (P, V)))
    t = r.integers(0, V, P).astype(np.uint16)
    t[[2, 5]] = 0
    grad, res = orc.cross_entropy_loss(x, t)
    xd = f32(x).astype(np.float64)
    valid = [i for i in range(P) if t[i] != 0]
    want_g = np.zeros_like(xd)
    loss = 0.0
    for i in valid:
        p = np.exp(xd[i] - xd[i].max())
        p /= p.sum()
        want_g[i] = p
        want_g[i, t[i]] -= 1
        loss -= np.log(p[t[i]])
    want_g /= len(valid)
    assert np.abs(f32(grad) - want_g).max() < 1e-3
    assert abs(f32(res)[0] - loss / len(valid)) < 1e-2 * (1 + loss / len(valid))


def test_causal_mask_and_sum_batch_closed_forms(orc):
    s = h(np.ones((3, 6, 6)))
    m = f32(orc.apply_causal_mask(s))
    i, j = np.indices((6, 6))
    assert np.all(m[:, j > i] == -65504) and np.all(m[:, j <= i] == 1)
    x = h(rng(9).integers(-8, 8, (5, 40)))
    out = f32(orc.sum_batch(x, h(np.full(40, 3)), 5, 40))
    assert np.array_equal(out, 3 + f32(x).sum(0))  # small integers: exact


def test_embed_backward_repeats_in_order(orc):
    """Repeated ids accumulate in index order with one fp16 rounding per add."""
    r = rng(10)
    idx = np.array([2, 0, 2, 2, 5, 0], np.uint16)
    gout = h(r.normal(0, 1, (6, 7)))
    base = h(r.normal(0, 1, (6, 7)))
    got = orc.embed_backward(gout, idx, base)
    want = f32(base).copy()
    for k, tok in enumerate(idx):
        want[tok] = (want[tok] + f32(gout)[k]).astype(np.float16).astype(np.float32)
    assert np.array_equal(f32(got), want)
    # ids past the table are skipped
    out_of_range = orc.embed_backward(gout[:1], np.array([9], np.uint16), base)
    assert np.array_equal(out_of_range, base)
