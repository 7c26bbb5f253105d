"""GPU parity: decode-step support ops (reference KATs + oracle) and the
KV-cached greedy decode model (identical greedy ids except at near-ties)."""
import numpy as np
import pytest

from conftest import assert_close_f16, f32, from_dev, to_dev

pytestmark = pytest.mark.gpu


def f16(x):
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def ulp_close(got, want, ulps=1):
    """fp16 results within `ulps` units in the last place (transcendental
    functions and reduction order differ between the GPU and glibc)."""
    g = got.astype(np.int32)
    w = want.astype(np.int32)
    gs = np.where(g & 0x8000, -(g & 0x7FFF), g)
    ws = np.where(w & 0x8000, -(w & 0x7FFF), w)
    return np.abs(gs - ws).max() <= ulps


def test_rms_norm(dev, orc):
    import evk_amd as evk
    import torch
    x = f16([[3, 4, 0, 0], [1, 2, 3, 4]])  # tests.h:1411-1444
    X = to_dev(x, dev)
    Y = torch.empty_like(X)
    evk.rms_norm(X, Y, 1e-4)
    torch.cuda.synchronize()
    assert ulp_close(from_dev(Y), orc.rms_norm(x, 1e-4))
    for shape in [(7, 768), (1, 3072), (33, 100)]:
        x = orc.normal_f16(shape, 301, 0, 2)
        X = to_dev(x, dev)
        Y = torch.empty_like(X)
        evk.rms_norm(X, Y, 1e-4)
        torch.cuda.synchronize()
        assert ulp_close(from_dev(Y), orc.rms_norm(x, 1e-4)), shape


def test_rope(dev, orc):
    import evk_amd as evk
    import torch
    x = f16([1, 2, 3, 4, 5, 6, 7, 8]).reshape(1, 2, 4)  # tests.h:1318-1356
    X = to_dev(x, dev)
    Y = torch.empty_like(X)
    evk.rope(X, Y, 1, 2, 4, 10000.0)
    torch.cuda.synchronize()
    assert ulp_close(from_dev(Y), orc.rope(x, 1, 2, 4, 10000.0))
    for (B, S, E, p0, hd) in [(2, 16, 64, 0, 0), (1, 1, 768, 1055, 64), (3, 5, 96, 17, 32)]:
        x = orc.normal_f16((B, S, E), 302 + E)
        X = to_dev(x, dev)
        Y = torch.empty_like(X)
        evk.rope(X, Y, B, S, E, 10000.0, p0, hd)
        torch.cuda.synchronize()
        want = orc.rope(x, B, S, E, 10000.0, p0, hd)
        assert_close_f16(from_dev(Y), want, atol=2e-3, rtol=2e-3, what="rope")


def test_gelu_add_embed(dev, orc):
    import evk_amd as evk
    import torch
    x = f16([-1.0, 0.0, 1.0])  # tests.h:1169-1190
    X = to_dev(x, dev)
    Y = torch.empty_like(X)
    evk.gelu(X, Y)
    torch.cuda.synchronize()
    assert ulp_close(from_dev(Y), orc.gelu(x))
    x = orc.normal_f16((3072,), 303, 0, 3)
    X = to_dev(x, dev)
    Y = torch.empty_like(X)
    evk.gelu(X, Y)
    torch.cuda.synchronize()
    assert ulp_close(from_dev(Y), orc.gelu(x))
    a, b = f16([0, 1, 2, 3]), f16([0, 2, 4, 6])  # tests.h:141-162
    A, B_ = to_dev(a, dev), to_dev(b, dev)
    C = torch.empty_like(A)
    evk.add(A, B_, C)
    torch.cuda.synchronize()
    assert np.array_equal(from_dev(C), f16([0, 3, 6, 9]))
    a, b = orc.normal_f16((1000,), 304), orc.normal_f16((1000,), 305)
    A, B_ = to_dev(a, dev), to_dev(b, dev)
    C = torch.empty_like(A)
    evk.add(A, B_, C)
    torch.cuda.synchronize()
    assert np.array_equal(from_dev(C), orc.add(a, b))
    table = f16(np.arange(1, 13)).reshape(4, 3)  # tests.h:1224-1252
    idx = np.array([1, 3], np.uint16)
    T = to_dev(table, dev)
    I = torch.from_numpy(idx.view(np.int16)).to(dev)
    O = torch.empty((2, 3), dtype=torch.float16, device=dev)
    evk.embed(T, I, O)
    torch.cuda.synchronize()
    assert np.array_equal(from_dev(O), table[[1, 3]])


def greedy_dev(evk, dev, logits, position, base, count):
    import torch
    L = to_dev(logits, dev)
    out = torch.zeros(logits.shape[0], dtype=torch.int16, device=dev)
    evk.greedy_sample(L, out, position, base, count)
    torch.cuda.synchronize()
    return from_dev(out)


def test_greedy_sample(dev, orc):
    import evk_amd as evk
    lp = np.full((2, 2, 5), f16(-10.0), np.uint16)  # tests.h:1472-1497
    lp[0, 1, 1:4] = f16([0.5, 2.5, 1.5])
    lp[1, 1, 1:4] = f16([3.0, 2.0, 1.0])
    assert list(greedy_dev(evk, dev, lp, 1, 1, 3)) == [2, 1]
    rs = np.random.RandomState(3)
    for trial in range(40):
        V = int(rs.choice([5, 256, 257, 1000, 32000]))
        pool = f16(rs.choice([-1.0, 0.0, -0.0, 0.5, 2.0, np.inf, -np.inf, np.nan], size=8))
        logits = pool[rs.randint(0, 8, size=(3, 2, V))]
        base = int(rs.randint(0, 3))
        count = int(rs.randint(0, V - base + 1))
        got = greedy_dev(evk, dev, logits, 1, base, count)
        want = orc.greedy_sample(logits, 1, base, count)
        assert np.array_equal(got, want), (trial, V, base, count)
    logits = orc.normal_f16((4, 1, 32000), 306)
    assert np.array_equal(greedy_dev(evk, dev, logits, 0, 0, 32000), orc.greedy_sample(logits, 0, 0, 32000))


# ---------------------------------------------------------------------------
# KV-cached decode model
# ---------------------------------------------------------------------------
def check_ids(got_ids, want_ids, logits_want):
    """Identical ids except where the oracle's top-2 logit gap is < 1e-3."""
    for s, (a, b) in enumerate(zip(got_ids, want_ids)):
        if a != b:
            top = np.sort(f32(logits_want[s]))[-2:]
            assert top[1] - top[0] < 1e-3, f"step {s}: got {a} want {b}"
            return s  # later steps follow a different token; stop comparing
    return None


def gpu_generate(evk, dev, cfg, w, prompt, steps, packed=False):
    """Prefill the prompt, then `steps` greedy steps; returns the steps+1 ids
    (first from the prefill), prefill logits, last logits and the cache.
    packed: the steps run through model_pack + model_decode_packed."""
    import torch
    W = to_dev(w, dev)
    cache = torch.zeros(evk.model_cache_elems(cfg), dtype=torch.float16, device=dev)
    feed = torch.from_numpy(prompt.view(np.int16)).to(dev)
    tok = torch.zeros(steps + 1, dtype=torch.int16, device=dev)
    logits = torch.empty(cfg.vocab, dtype=torch.float16, device=dev)
    evk.model_prefill(cfg, W, cache, feed, 0, tok, logits)
    torch.cuda.synchronize()
    first_logits = from_dev(logits).copy()
    if packed:
        P = torch.empty(evk.model_packed_elems(cfg), dtype=torch.float16, device=dev)
        evk.model_pack(cfg, W, P)
        evk.model_decode_packed(cfg, P, cache, tok, steps, len(prompt), logits)
    else:
        evk.model_decode(cfg, W, cache, tok, steps, len(prompt), logits)
    torch.cuda.synchronize()
    return from_dev(tok), first_logits, from_dev(logits), cache


def test_decode_small_model(dev, orc):
    import evk_amd as evk
    ocfg = orc.model_cfg(vocab=512, d=128, heads=2, layers=2, hidden=256, max_seq=96)
    cfg = evk.model_cfg(vocab=512, d=128, heads=2, layers=2, hidden=256, max_seq=96)
    w = orc.model_weights(ocfg, seed=311, std=0.1)
    prompt = orc.tokens_u16(40, 312, 512)
    ids, first_logits, last_logits, cache = gpu_generate(evk, dev, cfg, w, prompt, 20)
    want_ids, want_cache, want_logits = orc.model_generate(ocfg, w, prompt, 20, return_logits=True)
    assert_close_f16(first_logits, want_logits[0], what="prefill logits")
    stop = check_ids(list(ids), list(want_ids), want_logits)
    if stop is None:
        assert_close_f16(last_logits, want_logits[-1], what="last logits")
        assert_close_f16(from_dev(cache), want_cache, what="kv cache")


def test_decode_config4(dev, orc):
    """C4: 12 layers, d=768, 12x64 heads, hidden 3072, vocab 32000; prefill
    1024 seeded tokens, then 32 greedy steps; ids identical to the oracle's
    except at near-ties (top-2 gap < 1e-3)."""
    import evk_amd as evk
    ocfg = orc.model_cfg()
    cfg = evk.model_cfg()
    w = orc.model_weights(ocfg, seed=301, std=0.02)
    prompt = orc.tokens_u16(1024, 302, 32000)
    ids, first_logits, last_logits, _ = gpu_generate(evk, dev, cfg, w, prompt, 32)
    want_ids, _, want_logits = orc.model_generate(ocfg, w, prompt, 32, return_logits=True)
    assert_close_f16(first_logits, want_logits[0], what="prefill logits")
    stop = check_ids(list(ids), list(want_ids), want_logits)
    if stop is None:
        assert_close_f16(last_logits, want_logits[-1], what="step-32 logits")


@pytest.mark.parametrize("dims", [
    # (vocab, d, heads, layers, hidden, max_seq): head dims 16, 32, 64, 128,
    # ragged column blocks (3d and hidden not multiples of 128)
    [(512, 64, 4, 1, 96, 24), (1024, 256, 4, 2, 384, 40), (512, 64, 2, 2, 128, 16)],
    [(256, 128, 1, 1, 200, 12), (520, 96, 2, 2, 136, 70), (256, 128, 1, 1, 200, 12)],
])
def test_decode_workspace_reuse(dev, orc, dims):
    """Several model configurations in a row, smaller after larger: the
    library's grow-only decode workspace and its counters are reused."""
    import evk_amd as evk
    for (vocab, d, heads, layers, hidden, max_seq) in dims:
        kw = dict(vocab=vocab, d=d, heads=heads, layers=layers, hidden=hidden, max_seq=max_seq)
        ocfg, cfg = orc.model_cfg(**kw), evk.model_cfg(**kw)
        w = orc.model_weights(ocfg, seed=321 + d, std=0.1)
        steps = 4
        prompt = orc.tokens_u16(max_seq - steps - 1, 322 + d, vocab)
        ids, first_logits, last_logits, _ = gpu_generate(evk, dev, cfg, w, prompt, steps)
        want_ids, _, want_logits = orc.model_generate(ocfg, w, prompt, steps, return_logits=True)
        assert_close_f16(first_logits, want_logits[0], what=f"prefill logits {kw}")
        stop = check_ids(list(ids), list(want_ids), want_logits)
        if stop is None:
            assert_close_f16(last_logits, want_logits[-1], what=f"last logits {kw}")


# ---------------------------------------------------------------------------
# Persistent decode over packed weights (evkhip_model_pack /
# evkhip_model_decode_packed): same parity bar as model_decode.
# ---------------------------------------------------------------------------
def test_model_pack_layout(dev, orc):
    """Packed blob = E, then every matrix transposed to (out, in): bit-exact
    against numpy's transpose of the same blob."""
    import evk_amd as evk
    import torch
    kw = dict(vocab=520, d=96, heads=3, layers=2, hidden=136, max_seq=16)
    ocfg, cfg = orc.model_cfg(**kw), evk.model_cfg(**kw)
    w = orc.model_weights(ocfg, seed=341, std=0.1)
    P = torch.empty(evk.model_packed_elems(cfg), dtype=torch.float16, device=dev)
    evk.model_pack(cfg, to_dev(w, dev), P)
    torch.cuda.synchronize()
    got = from_dev(P)
    V, d, hid = 520, 96, 136
    want, o = [w[:V * d]], V * d
    for _ in range(2):
        for (k, n) in ((d, 3 * d), (d, d), (d, hid), (hid, d)):
            want.append(w[o:o + k * n].reshape(k, n).T.reshape(-1))
            o += k * n
    want.append(w[o:o + d * V].reshape(d, V).T.reshape(-1))
    assert np.array_equal(got, np.concatenate(want))


@pytest.mark.parametrize("kw,steps", [
    (dict(vocab=512, d=128, heads=2, layers=2, hidden=256, max_seq=96), 20),
    (dict(vocab=1024, d=256, heads=4, layers=3, hidden=512, max_seq=300), 12),  # several key splits
    (dict(vocab=256, d=64, heads=4, layers=1, hidden=96, max_seq=40), 8),       # dh 16
])
def test_decode_packed_small(dev, orc, kw, steps):
    import evk_amd as evk
    ocfg, cfg = orc.model_cfg(**kw), evk.model_cfg(**kw)
    w = orc.model_weights(ocfg, seed=351 + kw["d"], std=0.1)
    prompt = orc.tokens_u16(kw["max_seq"] - steps - 1, 352 + kw["d"], kw["vocab"])
    ids, first_logits, last_logits, cache = gpu_generate(evk, dev, cfg, w, prompt, steps, packed=True)
    want_ids, want_cache, want_logits = orc.model_generate(ocfg, w, prompt, steps, return_logits=True)
    assert evk.device_status(clear=True) == 0
    assert_close_f16(first_logits, want_logits[0], what="prefill logits")
    stop = check_ids(list(ids), list(want_ids), want_logits)
    if stop is None:
        assert_close_f16(last_logits, want_logits[-1], what="last logits")
        assert_close_f16(from_dev(cache), want_cache, what="kv cache")


def test_decode_config4_packed(dev, orc):
    """C4 through the persistent decode: 1024-token prefill, 32 greedy steps,
    ids identical to the oracle's except at near-ties."""
    import evk_amd as evk
    ocfg, cfg = orc.model_cfg(), evk.model_cfg()
    w = orc.model_weights(ocfg, seed=301, std=0.02)
    prompt = orc.tokens_u16(1024, 302, 32000)
    ids, first_logits, last_logits, _ = gpu_generate(evk, dev, cfg, w, prompt, 32, packed=True)
    want_ids, _, want_logits = orc.model_generate(ocfg, w, prompt, 32, return_logits=True)
    assert evk.device_status(clear=True) == 0
    stop = check_ids(list(ids), list(want_ids), want_logits)
    if stop is None:
        assert_close_f16(last_logits, want_logits[-1], what="step-32 logits")


def test_decode_packed_repeated_and_replayed(dev, orc):
    """The same steps three times in a row (each launch takes new hand-over
    tags from the device), then captured into a HIP graph and replayed twice
    with eager launches in between: identical ids and logits every time."""
    import evk_amd as evk
    import torch
    kw = dict(vocab=512, d=128, heads=2, layers=2, hidden=256, max_seq=64)
    ocfg, cfg = orc.model_cfg(**kw), evk.model_cfg(**kw)
    w = orc.model_weights(ocfg, seed=361, std=0.1)
    prompt = orc.tokens_u16(40, 362, 512)
    W = to_dev(w, dev)
    cache = torch.zeros(evk.model_cache_elems(cfg), dtype=torch.float16, device=dev)
    tok = torch.zeros(9, dtype=torch.int16, device=dev)
    logits = torch.empty(cfg.vocab, dtype=torch.float16, device=dev)
    evk.model_prefill(cfg, W, cache, torch.from_numpy(prompt.view(np.int16)).to(dev), 0, tok, logits)
    P = torch.empty(evk.model_packed_elems(cfg), dtype=torch.float16, device=dev)
    evk.model_pack(cfg, W, P)
    torch.cuda.synchronize()
    first = tok[0].clone()

    def run():
        tok[0] = first
        evk.model_decode_packed(cfg, P, cache, tok, 8, 40, logits)

    run()
    torch.cuda.synchronize()
    want_tok, want_lg = tok.clone(), logits.clone()
    for _ in range(2):
        run()
        torch.cuda.synchronize()
        assert torch.equal(tok, want_tok) and torch.equal(logits, want_lg)
    g = torch.cuda.CUDAGraph()
    try:
        with torch.cuda.graph(g):
            run()
    except Exception as ex:
        pytest.fail(f"graph capture of the persistent launch failed: {ex}")
    for _ in range(2):
        tok.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(tok, want_tok) and torch.equal(logits, want_lg)
        run()
        torch.cuda.synchronize()
        assert torch.equal(tok, want_tok) and torch.equal(logits, want_lg)
    assert evk.device_status(clear=True) == 0


def test_decode_packed_tag_wrap(dev, orc):
    """The hand-over tags wrap: launches near the end of the tag range clear
    the mailboxes and restart the tags from zero behind a barrier of every
    workgroup.  Set just below the wrap point, a launch that still fits, one
    that wraps, and the ones after it give the same ids and logits as a
    launch far from it, and none reports a wait timeout."""
    import evk_amd as evk
    import torch
    kw = dict(vocab=512, d=128, heads=2, layers=2, hidden=256, max_seq=64)
    ocfg, cfg = orc.model_cfg(**kw), evk.model_cfg(**kw)
    w = orc.model_weights(ocfg, seed=371, std=0.1)
    prompt = orc.tokens_u16(40, 372, 512)
    W = to_dev(w, dev)
    cache = torch.zeros(evk.model_cache_elems(cfg), dtype=torch.float16, device=dev)
    tok = torch.zeros(9, dtype=torch.int16, device=dev)
    logits = torch.empty(cfg.vocab, dtype=torch.float16, device=dev)
    evk.model_prefill(cfg, W, cache, torch.from_numpy(prompt.view(np.int16)).to(dev), 0, tok, logits)
    P = torch.empty(evk.model_packed_elems(cfg), dtype=torch.float16, device=dev)
    evk.model_pack(cfg, W, P)
    torch.cuda.synchronize()
    first = tok[0].clone()

    def run():
        tok[0] = first
        evk.model_decode_packed(cfg, P, cache, tok, 8, 40, logits)
        torch.cuda.synchronize()
        return tok.clone(), logits.clone()

    evk.device_status(clear=True)
    want_tok, want_lg = run()
    # a launch takes 8 steps x (5 stages x 2 layers + the head) + 2 = 90 tags
    need = 8 * (5 * 2 + 1) + 2
    for distance in (need + 1, 1):  # first a launch that fits, then one that wraps at once
        evk.debug_decode_set_epoch(distance)
        for _ in range(3):
            t, lg = run()
            assert torch.equal(t, want_tok) and torch.equal(lg, want_lg), f"distance {distance}"
    assert evk.device_status(clear=True) == 0


def test_decode_packed_wait_timeout_is_reported(dev, orc):
    """A spin limit of one round (set from the host) makes the persistent
    decode's hand-over waits give up: every workgroup leaves, the call's
    status raises EVKHIP_STATUS_WAIT_TIMEOUT, and the next call with the
    default limit is correct again (it takes new tags)."""
    import evk_amd as evk
    import torch
    kw = dict(vocab=512, d=128, heads=2, layers=2, hidden=256, max_seq=64)
    ocfg, cfg = orc.model_cfg(**kw), evk.model_cfg(**kw)
    w = orc.model_weights(ocfg, seed=371, std=0.1)
    prompt = orc.tokens_u16(40, 372, 512)
    want_ids, _, want_logits = orc.model_generate(ocfg, w, prompt, 6, return_logits=True)
    W = to_dev(w, dev)
    cache = torch.zeros(evk.model_cache_elems(cfg), dtype=torch.float16, device=dev)
    tok = torch.zeros(7, dtype=torch.int16, device=dev)
    logits = torch.empty(cfg.vocab, dtype=torch.float16, device=dev)
    evk.model_prefill(cfg, W, cache, torch.from_numpy(prompt.view(np.int16)).to(dev), 0, tok, logits)
    P = torch.empty(evk.model_packed_elems(cfg), dtype=torch.float16, device=dev)
    evk.model_pack(cfg, W, P)
    torch.cuda.synchronize()
    first = tok[0].clone()
    evk.device_status(clear=True)
    try:
        evk.debug_set_spin_limit(1)
        evk.model_decode_packed(cfg, P, cache, tok, 6, 40, logits)
        torch.cuda.synchronize()
        forced = evk.device_status(clear=True)
    finally:
        evk.debug_set_spin_limit(0)
    assert forced & evk.STATUS_WAIT_TIMEOUT
    tok[0] = first
    evk.model_decode_packed(cfg, P, cache, tok, 6, 40, logits)
    torch.cuda.synchronize()
    assert evk.device_status(clear=True) == 0
    stop = check_ids(list(from_dev(tok)), list(want_ids), want_logits)
    if stop is None:
        assert_close_f16(from_dev(logits), want_logits[-1], what="last logits after a timeout")


def test_prefill_in_two_parts(dev, orc):
    """A prompt prefilled in two calls: the first part from position 0 runs as
    whole-sequence ops (batched GEMMs, causal flash per head), the second part
    at pos0 > 0 through the token loop.  The cache, the logits after the last
    prompt token and the next id match the oracle's single prefill (ids
    except at near-ties)."""
    import torch
    import evk_amd as evk
    kw = dict(vocab=512, d=128, heads=2, layers=2, hidden=256, max_seq=96)
    ocfg, cfg = orc.model_cfg(**kw), evk.model_cfg(**kw)
    w = orc.model_weights(ocfg, seed=361, std=0.1)
    prompt = orc.tokens_u16(70, 362, kw["vocab"])
    W = to_dev(w, dev)
    cache = torch.zeros(evk.model_cache_elems(cfg), dtype=torch.float16, device=dev)
    tok = torch.zeros(2, dtype=torch.int16, device=dev)
    logits = torch.empty(cfg.vocab, dtype=torch.float16, device=dev)
    feed = torch.from_numpy(prompt.view(np.int16)).to(dev)
    evk.model_prefill(cfg, W, cache, feed[:48], 0, tok, logits)
    evk.model_prefill(cfg, W, cache, feed[48:], 48, tok, logits)
    torch.cuda.synchronize()
    want_ids, want_cache, want_logits = orc.model_generate(ocfg, w, prompt, 0, return_logits=True)
    assert_close_f16(from_dev(logits), want_logits[0], what="logits after the prompt")
    stop = check_ids([int(from_dev(tok)[0])], [int(want_ids[0])], want_logits)
    if stop is None:
        assert_close_f16(from_dev(cache), want_cache, what="kv cache")
