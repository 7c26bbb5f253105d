"""GPU parity: evk::ai::matmul through the C ABI vs the CPU oracle.

Bar: fp16 outputs within max-abs/relative 1e-2 of the fp32-accumulated
oracle; known-answer tests bit-exact (reference tests.h:163-219).
"""
import numpy as np
import pytest

from conftest import assert_close_f16, f32, from_dev, to_dev

pytestmark = pytest.mark.gpu


def f16(x):
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def run_mm(evk, dev, a, b, c_shape, ta=False, tb=False, acc=False, c0=None, tiles=(80, 80)):
    import torch
    A, B = to_dev(a, dev), to_dev(b, dev)
    C = to_dev(c0, dev) if c0 is not None else torch.zeros(c_shape, dtype=torch.float16, device=dev)
    evk.matmul(A, B, C, ta, tb, acc, *tiles)
    torch.cuda.synchronize()
    return from_dev(C)


def test_identity_kat_400(dev, orc):
    # tests.h:163-194 with the default 80x80 tile hints
    import evk_amd as evk
    n = 400
    eye2 = np.zeros((n, n), np.uint16)
    eye2[np.arange(n), np.arange(n)] = f16(2.0)
    c = run_mm(evk, dev, eye2, eye2, (n, n))
    want = np.zeros((n, n), np.uint16)
    want[np.arange(n), np.arange(n)] = f16(4.0)
    assert np.array_equal(c, want)


def test_broadcast_kat(dev, orc):
    # tests.h:196-219: a (1,32,32) ones, b (32,32) identity, c (3,32,32)
    import evk_amd as evk
    ones = np.full((1, 32, 32), f16(1.0), np.uint16)
    eye = np.zeros((32, 32), np.uint16)
    eye[np.arange(32), np.arange(32)] = f16(1.0)
    c = run_mm(evk, dev, ones, eye, (3, 32, 32), tiles=(16, 16))
    assert np.all(c == f16(1.0))


def test_config1_gemm_1024(dev, orc):
    import evk_amd as evk
    a = orc.uniform_f16((1024, 1024), 101)
    b = orc.uniform_f16((1024, 1024), 102)
    got = run_mm(evk, dev, a, b, (1024, 1024))
    assert_close_f16(got, orc.matmul(a, b), what="C1 1024^3")


@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
@pytest.mark.parametrize("M,N,K", [(200, 136, 72), (64, 64, 64), (520, 264, 328), (32, 8, 8)])
def test_transposes_ragged(dev, orc, ta, tb, M, N, K):
    import evk_amd as evk
    a = orc.uniform_f16((K, M) if ta else (M, K), 11 + M)
    b = orc.uniform_f16((N, K) if tb else (K, N), 12 + N)
    got = run_mm(evk, dev, a, b, (M, N), ta, tb)
    assert_close_f16(got, orc.matmul(a, b, transpose_a=ta, transpose_b=tb), what=f"{ta}{tb} {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K", [(600, 1100, 968), (1536, 1536, 256)])
def test_large_tile_paths(dev, orc, M, N, K):
    import evk_amd as evk
    a = orc.uniform_f16((M, K), 41)
    b = orc.uniform_f16((K, N), 42)
    got = run_mm(evk, dev, a, b, (M, N))
    assert_close_f16(got, orc.matmul(a, b), what=f"{M}x{N}x{K}")


@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
def test_k_groups_ragged(dev, orc, ta, tb):
    """Grids that fit the CUs once with a long K (64x64 tiles, K >= 1024) run
    four K groups per workgroup whose sums meet in LDS: ragged M, N and a K
    that is not a multiple of the 64-deep tile (the last group's range is
    shorter), every operand order."""
    import evk_amd as evk
    M, N, K = 200, 136, 1096
    a = orc.uniform_f16((K, M) if ta else (M, K), 61 + ta)
    b = orc.uniform_f16((N, K) if tb else (K, N), 62 + tb)
    got = run_mm(evk, dev, a, b, (M, N), ta, tb)
    assert_close_f16(got, orc.matmul(a, b, transpose_a=ta, transpose_b=tb), what=f"K groups {ta}{tb}")


def test_k_groups_batched_acc(dev, orc):
    """K groups with accumulation into C (one rounding of the fp32 sum per
    element) over a batch."""
    import evk_amd as evk
    a = orc.uniform_f16((3, 96, 2056), 63)
    b = orc.uniform_f16((2056, 72), 64)
    c0 = orc.uniform_f16((3, 96, 72), 65)
    got = run_mm(evk, dev, a, b, None, acc=True, c0=c0)
    assert_close_f16(got, orc.matmul(a, b, c=c0, acc_c=True), what="K groups batched acc")


def test_batched_broadcast_acc(dev, orc):
    import evk_amd as evk
    a = orc.uniform_f16((3, 96, 80), 51)
    b = orc.uniform_f16((80, 48), 52)
    c0 = orc.uniform_f16((3, 96, 48), 53)
    got = run_mm(evk, dev, a, b, None, acc=True, c0=c0)
    assert_close_f16(got, orc.matmul(a, b, c=c0, acc_c=True), what="batched acc")
    # broadcast A over a batched B, transposed B
    a1 = orc.uniform_f16((40, 64), 54)
    b3 = orc.uniform_f16((2, 24, 64), 55)
    got = run_mm(evk, dev, a1, b3, (2, 40, 24), tb=True)
    want = orc.matmul(a1, b3, transpose_b=True, out_shape=(2, 40, 24))
    assert_close_f16(got, want, what="broadcast A")


def test_unaligned_fallback(dev, orc):
    import evk_amd as evk
    a = orc.uniform_f16((13, 7), 61)
    b = orc.uniform_f16((7, 5), 62)
    got = run_mm(evk, dev, a, b, (13, 5))
    assert_close_f16(got, orc.matmul(a, b), what="scalar path")


@pytest.mark.parametrize("M", [1, 4, 16])
def test_skinny_gemv_config5(dev, orc, M):
    import evk_amd as evk
    K, N = 4096, 11008
    a = orc.uniform_f16((M, K), 501 + M)
    b = orc.uniform_f16((K, N), 510)
    got = run_mm(evk, dev, a, b, (M, N))
    assert_close_f16(got, orc.matmul(a, b), what=f"gemv M={M}")
    # second call reuses the split-K workspace: must give identical bits
    got2 = run_mm(evk, dev, a, b, (M, N))
    assert np.array_equal(got, got2)


def test_skinny_acc_and_small(dev, orc):
    import evk_amd as evk
    # M <= 4 runs on the VALU kernel, 4 < M <= 16 on the MFMA one; K ranges of
    # 512 rows: single-range (direct C write) and ragged split-K cases
    for (M, K, N) in [(1, 768, 2304), (3, 3072, 768), (2, 8, 16), (1, 4096, 32000),
                      (5, 512, 64), (8, 1000, 136), (16, 520, 2000), (12, 4096, 1032), (9, 24, 40)]:
        a = orc.uniform_f16((M, K), 71 + K)
        b = orc.uniform_f16((K, N), 72 + N)
        c0 = orc.uniform_f16((M, N), 73)
        got = run_mm(evk, dev, a, b, None, acc=True, c0=c0)
        assert_close_f16(got, orc.matmul(a, b, c=c0, acc_c=True), what=f"gemv acc {M}x{K}x{N}")


def test_skinny_batched(dev, orc):
    """Batched skinny products: per-batch A over a shared B (MFMA kernel,
    split-K), and a shared A over per-batch B (VALU kernel)."""
    import evk_amd as evk
    a = orc.uniform_f16((3, 12, 1040), 81)
    b = orc.uniform_f16((1040, 200), 82)
    got = run_mm(evk, dev, a, b, (3, 12, 200))
    assert_close_f16(got, orc.matmul(a, b, out_shape=(3, 12, 200)), what="batched A")
    a1 = orc.uniform_f16((1, 520), 83)
    b3 = orc.uniform_f16((2, 520, 72), 84)
    got = run_mm(evk, dev, a1, b3, (2, 1, 72))
    assert_close_f16(got, orc.matmul(a1, b3, out_shape=(2, 1, 72)), what="batched B")


def _rows_check(orc, a, b, got, rows):
    want = orc.matmul(a[rows], b)
    assert_close_f16(got[rows], want, what="row sample")


def half_ulp(x):
    """Half an fp16 ulp of each |x| (the rounding bound of the fp16 store)."""
    ax = np.maximum(np.abs(x.astype(np.float64)), 2.0 ** -14)
    return 0.5 * 2.0 ** (np.floor(np.log2(ax)) - 10)


def test_config5_square_4096(dev, orc):
    import evk_amd as evk
    n = 4096
    a = orc.uniform_f16((n, n), 501)
    b = orc.uniform_f16((n, n), 502)
    got = run_mm(evk, dev, a, b, (n, n))
    rows = np.random.RandomState(0).choice(n, 48, replace=False)
    _rows_check(orc, a, b, got, np.sort(rows))
    # checksum over every row: C.1 == A.(B.1) up to the fp16 rounding of each
    # stored element (bounded by half an ulp) plus fp32 accumulation slack
    A, B = f32(a).astype(np.float64), f32(b).astype(np.float64)
    G = f32(got)
    err = np.abs(G.astype(np.float64).sum(1) - A @ B.sum(1))
    bound = half_ulp(G).sum(1) + 1e-2 * np.sqrt(n)
    assert np.all(err <= bound), float((err - bound).max())


def test_config5_qkv_shape(dev, orc):
    import evk_amd as evk
    M, N, K = 8192, 12288, 4096
    a = orc.uniform_f16((M, K), 503)
    b = orc.uniform_f16((K, N), 504)
    got = run_mm(evk, dev, a, b, (M, N))
    rows = np.sort(np.random.RandomState(1).choice(M, 16, replace=False))
    _rows_check(orc, a, b, got, rows)
    A, B = f32(a).astype(np.float64), f32(b).astype(np.float64)
    G = f32(got)
    err = np.abs(G.astype(np.float64).sum(0) - A.sum(0) @ B)
    bound = half_ulp(G).sum(0) + 1e-2 * np.sqrt(M)
    assert np.all(err <= bound), float((err - bound).max())


@pytest.mark.parametrize("ta", [False, True])
def test_operand_over_2gib_takes_tiled_path(dev, orc, ta):
    """A 2.15 GB A operand (past the 32-bit buffer-descriptor range of the
    MFMA kernel) runs the 64-bit-addressed tiled kernel; sampled rows of C and
    whole-matrix column sums are checked against fp32 on the host.  Inputs
    are drawn on the device from a seeded torch generator (2 GB is too much
    to push from the host in a test)."""
    import torch
    import evk_amd as evk
    M, K, N = 131072 + 64, 8192, 256
    assert M * K * 2 > 2**31
    g = torch.Generator(device=dev).manual_seed(7)
    shape_a = (K, M) if ta else (M, K)
    A = (torch.rand(shape_a, generator=g, device=dev, dtype=torch.float16) * 2 - 1)
    B = (torch.rand((K, N), generator=g, device=dev, dtype=torch.float16) * 2 - 1)
    C = torch.empty((M, N), dtype=torch.float16, device=dev)
    evk.matmul(A, B, C, ta, False, False)
    torch.cuda.synchronize()
    rows = torch.tensor([0, 1, 255, 256, 70000, M // 2 + 3, M - 65, M - 1], device=dev)
    a_rows = (A[:, rows].t() if ta else A[rows]).float().cpu().numpy()
    want = a_rows @ B.float().cpu().numpy()
    got = C[rows].float().cpu().numpy()
    assert np.abs(got - want).max() <= 1e-2 * (1 + np.abs(want).max())
    # every row: column sums of C against (column sums of A) . B
    a_sum = (A.float().sum(dim=1) if ta else A.float().sum(dim=0)).cpu().numpy()
    want_cs = a_sum @ B.float().cpu().numpy()
    got_cs = C.float().sum(dim=0).cpu().numpy()
    assert np.abs(got_cs - want_cs).max() <= 2e-3 * np.abs(want_cs).max() + 1.0
    del A, B, C
    torch.cuda.empty_cache()
