"""evkhip_matmul_noalloc (no reference counterpart: the entry point for
callers that cannot allocate) against evkhip_matmul, through the C ABI.

Both run the same kernels, so the outputs must be bit-identical; two calls in
a row (the second smaller, with acc) check that the shared static scratch is
reused correctly, and an oversized split-K request must fail before any
launch.  Results are also held against the CPU oracle."""
import ctypes as C

import numpy as np
import pytest

from conftest import assert_close_f16, from_dev, to_dev

pytestmark = pytest.mark.gpu


def _call(fn, A, B, Cd, ta=0, tb=0, acc=0):
    import torch
    import evk_amd as evk
    rc = fn(C.byref(evk.desc(A)), C.byref(evk.desc(B)), C.byref(evk.desc(Cd)), ta, tb, acc, 80, 80,
            C.c_void_p(torch.cuda.current_stream().cuda_stream))
    return rc


@pytest.mark.parametrize("first,second", [((16, 11008, 4096), (4, 4096, 2048)),
                                          ((8, 4096, 4096), (1, 1024, 1536))])
def test_noalloc_matches_matmul_twice(dev, orc, first, second):
    import torch
    import evk_amd as evk
    L = evk.lib()
    for i, (M, N, K) in enumerate((first, second)):
        a = orc.uniform_f16((M, K), 601 + 7 * i + M)
        b = orc.uniform_f16((K, N), 602 + 7 * i + N)
        A, B = to_dev(a, dev), to_dev(b, dev)
        acc = i == 1
        c0 = orc.uniform_f16((M, N), 603 + i)
        C_ref = to_dev(c0, dev)
        C_na = to_dev(c0, dev)
        assert _call(L.evkhip_matmul, A, B, C_ref, acc=int(acc)) == 0
        assert _call(L.evkhip_matmul_noalloc, A, B, C_na, acc=int(acc)) == 0, L.evkhip_last_error()
        torch.cuda.synchronize()
        got, want = from_dev(C_na), from_dev(C_ref)
        assert np.array_equal(got, want), f"call {i} ({M}x{N}x{K}) differs from evkhip_matmul"
        assert_close_f16(got, orc.matmul(a, b, c=c0, acc_c=acc), what=f"noalloc call {i}")


def test_noalloc_mfma_path_and_oversize(dev, orc):
    import torch
    import evk_amd as evk
    L = evk.lib()
    a = orc.uniform_f16((256, 512), 611)
    b = orc.uniform_f16((512, 384), 612)
    A, B = to_dev(a, dev), to_dev(b, dev)
    C1 = torch.zeros((256, 384), dtype=torch.float16, device=dev)
    C2 = torch.zeros_like(C1)
    assert _call(L.evkhip_matmul, A, B, C1) == 0
    assert _call(L.evkhip_matmul_noalloc, A, B, C2) == 0
    torch.cuda.synchronize()
    assert np.array_equal(from_dev(C1), from_dev(C2))
    # split-K partials of 32 x 16 x 11008 fp32 exceed the 8 MiB of scratch:
    # rejected on the host, nothing launched (B is never read)
    A = torch.zeros((16, 16384), dtype=torch.float16, device=dev)
    B = torch.empty((16384, 11008), dtype=torch.float16, device=dev)
    Cd = torch.zeros((16, 11008), dtype=torch.float16, device=dev)
    assert _call(L.evkhip_matmul_noalloc, A, B, Cd) == -3  # EVKHIP_ERR_UNSUPPORTED
    assert b"scratch" in L.evkhip_last_error()
    torch.cuda.synchronize()
    assert not Cd.any()
