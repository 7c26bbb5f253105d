"""CPU-only checks of the C ABI boundary: the library loads, exports every
entry point include/*.h declares, and rejects malformed calls with the
documented status codes before touching the GPU (no compute calls here)."""
import ctypes as C
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

OK, INVALID, SHAPE, UNSUPPORTED = 0, -1, -2, -3


def declared(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(evkhip_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def L():
    import evk_amd
    if not evk_amd.available():
        pytest.fail("libevkhip.so is not built: run `python -m evk_amd.build`")
    return evk_amd.lib()


def test_exports_every_declared_symbol(L):
    import evk_amd
    names = declared("evkhip.h")
    assert len(names) >= 18
    for n in names:
        assert hasattr(L, n), f"libevkhip.so does not export {n}"
        assert n in evk_amd.SIGNATURES, f"Python mirror lacks a signature for {n}"
    assert set(evk_amd.SIGNATURES) == set(names)


def test_api_library_exports(L):
    path = os.path.join(ROOT, "evk_amd", "libevk.so")
    if not os.path.exists(path):
        pytest.fail("libevk.so (the evk::ai C++ API) is not built")
    api = C.CDLL(path)
    # a few mangled evk::ai entry points the C++ callers link against
    syms = os.popen(f"nm -D --defined-only {path}").read()
    for needle in ["ai6matmul", "ai15flash_attention", "ai19flash_attention_bwd",
                   "ai22single_query_attention", "ai8rms_norm", "ai4rope", "ai13greedy_sample",
                   "ai10initialize", "ai8shutdown", "CreateBuffer", "CmdBegin", "CmdWait"]:
        assert needle in syms, needle
    del api


def _api_tests_binary():
    exe = os.path.join(ROOT, "evk_amd", "bin", "api_tests")
    if not os.path.exists(exe):
        pytest.fail("evk_amd/bin/api_tests is not built: run `python -m evk_amd.build`")
    return exe


def test_cpp_api_host_tests():
    # float16_t and Shape of include/evk_ai.h, no GPU calls
    import subprocess
    r = subprocess.run([_api_tests_binary(), "--cpu"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "ALL PASSED" in r.stdout, r.stdout[-2000:] + r.stderr[-2000:]


def test_cpp_float16_matches_oracle(tmp_path, orc):
    # the header's fp32->fp16 conversion bit-equals the oracle's (itself
    # pinned to the reference's float16_t) on 2^20 patterns over all exponents
    import subprocess

    import numpy as np
    out = tmp_path / "f16.bin"
    r = subprocess.run([_api_tests_binary(), "--f16-sweep", str(out)], capture_output=True, timeout=120)
    assert r.returncode == 0
    got = np.fromfile(out, dtype=np.uint16)
    bits = (np.arange(1 << 20, dtype=np.uint64) * 4093).astype(np.uint32)
    want = orc.f32_to_f16(bits.view(np.float32))
    assert got.shape == want.shape
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(hex(int(bits[i])), hex(int(got[i])), hex(int(want[i]))) for i in bad[:5]]


def T(shape, ptr=0x1000):
    import evk_amd
    return evk_amd.desc((ptr, tuple(shape)))


def call(L, name, *args):
    return getattr(L, name)(*args)


def test_version_and_errors(L):
    assert L.evkhip_version().startswith(b"evkhip")
    r = L.evkhip_matmul(None, None, None, 0, 0, 0, 80, 80, None)
    assert r == INVALID
    assert b"null" in L.evkhip_last_error()


def test_matmul_validation(L):
    b = C.byref
    # inner dimensions differ
    assert L.evkhip_matmul(b(T((4, 8))), b(T((9, 4))), b(T((4, 4))), 0, 0, 0, 80, 80, None) == SHAPE
    # output shape wrong
    assert L.evkhip_matmul(b(T((4, 8))), b(T((8, 4))), b(T((4, 5))), 0, 0, 0, 80, 80, None) == SHAPE
    # transposes change the logical dims: A (8,4)^T . B (4,8)^T needs C (4,4)
    assert L.evkhip_matmul(b(T((8, 4))), b(T((4, 8))), b(T((4, 5))), 1, 1, 0, 80, 80, None) == SHAPE
    # batch mismatch (evk_ai.cpp:266-268)
    assert L.evkhip_matmul(b(T((2, 4, 8))), b(T((3, 8, 4))), b(T((3, 4, 4))), 0, 0, 0, 80, 80, None) == SHAPE
    # C batch must equal the broadcast batch
    assert L.evkhip_matmul(b(T((2, 4, 8))), b(T((8, 4))), b(T((4, 4))), 0, 0, 0, 80, 80, None) == SHAPE
    # tile hints must be multiples of 16
    assert L.evkhip_matmul(b(T((4, 8))), b(T((8, 4))), b(T((4, 4))), 0, 0, 0, 40, 80, None) == INVALID
    # rank 1 is not a matrix
    assert L.evkhip_matmul(b(T((8,))), b(T((8, 4))), b(T((4,))), 0, 0, 0, 80, 80, None) == SHAPE
    # empty output: a valid no-op, returns before any launch
    assert L.evkhip_matmul(b(T((0, 8))), b(T((8, 4))), b(T((0, 4))), 0, 0, 0, 80, 80, None) == OK


def test_flash_validation(L):
    b = C.byref
    q, k = T((2, 16, 128)), T((2, 16, 64))
    assert L.evkhip_flash_attention(b(q), b(k), b(k), b(T((2, 16, 64))), 0, None, None) == SHAPE
    assert L.evkhip_flash_attention(b(q), b(T((2, 15, 64))), b(k), b(q), 0, None, None) == SHAPE
    assert L.evkhip_flash_attention(b(q), b(T((2, 16, 48))), b(T((2, 16, 48))), b(q), 0, None, None) == SHAPE
    assert L.evkhip_flash_attention(b(T((2, 16, 1024))), b(T((2, 16, 512))), b(T((2, 16, 512))),
                                    b(T((2, 16, 1024))), 0, None, None) == UNSUPPORTED
    # heads must equal D/Dh when given (evk_ai.cpp:393-395)
    args = [b(q), b(k), b(k), b(q), b(q), b(q), b(k), b(k)]
    assert L.evkhip_flash_attention_bwd(*args, 3, 0, None, None) == SHAPE
    bad = [b(q), b(k), b(k), b(q), b(q), b(q), b(q), b(k)]
    assert L.evkhip_flash_attention_bwd(*bad, 0, 0, None, None) == SHAPE
    assert L.evkhip_flash_attention(b(T((0, 16, 128))), b(T((0, 16, 64))), b(T((0, 16, 64))),
                                    b(T((0, 16, 128))), 1, None, None) == OK


def test_flash_kernel_path(L):
    """The wide-head MFMA kernels address one batch of Q through 32-bit buffer
    offsets: at 2 GiB and above the dispatch takes the scalar kernels."""
    SCALAR, MFMA, WIDE = 0, 1, 2
    for dh in (32, 64, 128):
        assert L.evkhip_flash_kernel_path(1024, 8, dh) == MFMA
    for dh in (16, 48, 80, 96, 160, 256):
        assert L.evkhip_flash_kernel_path(1024, 8, dh) == WIDE
    for dh in (8, 24, 100, 0):
        assert L.evkhip_flash_kernel_path(1024, 8, dh) == SCALAR
    # N * H * dh * 2 bytes against INT32_MAX
    lim = (2**31 - 1)
    n = lim // (2 * 256)  # 4194303 rows of head 256: just below
    assert n * 256 * 2 < lim
    assert L.evkhip_flash_kernel_path(n, 1, 256) == WIDE
    assert L.evkhip_flash_kernel_path(n + 1, 1, 256) == SCALAR
    assert L.evkhip_flash_kernel_path(1 << 22, 8, 48) == SCALAR  # 3.2 GB of Q per batch
    assert L.evkhip_flash_kernel_path(1 << 22, 1, 48) == WIDE    # 403 MB
    assert L.evkhip_flash_kernel_path(1 << 30, 1, 64) == MFMA  # these pick a sub-kernel by size themselves


def test_decode_op_validation(L):
    b = C.byref
    q, kc = T((768,)), T((1056, 768))
    assert L.evkhip_single_query_attention(b(q), b(kc), b(kc), b(q), 1057, 12, None) == SHAPE
    assert L.evkhip_single_query_attention(b(q), b(kc), b(kc), b(q), 10, 0, None) == INVALID
    assert L.evkhip_single_query_attention(b(q), b(kc), b(kc), b(q), 10, 7, None) == SHAPE
    assert L.evkhip_single_query_attention(b(q), b(T((1056, 512))), b(T((1056, 512))), b(q), 10, 12,
                                           None) == SHAPE
    assert L.evkhip_rms_norm(b(T((4, 8))), b(T((4, 9))), C.c_float(1e-4), None) == SHAPE
    assert L.evkhip_rope(b(T((1, 2, 5))), b(T((1, 2, 5))), 1, 2, 5, C.c_float(1e4), 0, 0, None) == SHAPE
    assert L.evkhip_rope(b(T((1, 2, 12))), b(T((1, 2, 12))), 1, 2, 12, C.c_float(1e4), 0, 5, None) == SHAPE
    assert L.evkhip_rope(b(T((1, 2, 8))), b(T((1, 2, 8))), 1, 3, 8, C.c_float(1e4), 0, 0, None) == SHAPE
    assert L.evkhip_gelu(b(T((3,))), b(T((4,))), None) == SHAPE
    assert L.evkhip_add(b(T((3,))), b(T((3,))), b(T((4,))), None) == SHAPE
    assert L.evkhip_embed(b(T((4, 3))), b(T((2,))), b(T((2, 4))), None) == SHAPE
    lg = T((2, 3, 10))
    assert L.evkhip_greedy_sample(b(lg), b(T((3,))), 0, 0, 10, None) == SHAPE
    assert L.evkhip_greedy_sample(b(lg), b(T((2,))), 3, 0, 10, None) == SHAPE
    assert L.evkhip_greedy_sample(b(lg), b(T((2,))), 0, 5, 6, None) == SHAPE


def test_model_validation(L):
    import evk_amd
    cfg = evk_amd.model_cfg()
    assert evk_amd.model_weight_elems(cfg) == (32000 * 768 + 12 * (768 * 2304 + 768 * 768 + 2 * 768 * 3072)
                                               + 768 * 32000)
    assert evk_amd.model_cache_elems(cfg) == 12 * 2 * 1056 * 768
    p = C.c_void_p(0x1000)
    # positions beyond max_seq
    r = L.evkhip_model_decode(C.byref(cfg), p, p, p, 40, 1040, p, None)
    assert r == SHAPE
    bad = evk_amd.ModelCfg(32000, 768, 12, 60, 12, 3072, 1056, 1e-4, 1e4)  # heads*dh != d
    assert L.evkhip_model_decode(C.byref(bad), p, p, p, 1, 0, p, None) == SHAPE
    assert L.evkhip_model_prefill(C.byref(cfg), p, p, None, 4, 0, p, p, None) == INVALID
