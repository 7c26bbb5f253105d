"""evk::ai::KVCacheDecoder at the shape of the reference's own sampling loop
(example/main_llm.cpp:622-654, model :528-546, sizes :694-702: B=16
sequences, D=256 as one head, hidden 512, 8 layers, vocab 144) against the
CPU oracle's decode model (oracle/oracle.c orc_model_forward, with heads=1,
dh=256).

tests/cpp/kv_decoder_tool.cpp builds the model with the reference's
initialisation, prefills an 18-token prompt per sequence and runs 32 greedy
steps over the coordinate-token range [3, 131), each sequence fed its own
ids; it writes the weights (in the oracle's blob layout), the prompts, the
logits of every step and the sampled ids.  Every sequence is then replayed
through the oracle with the same ids: logits within 1e-2 (abs + rel), and
every id equal to the oracle's argmax over the range except where the
oracle's two logits differ by less than 1e-3."""
import ctypes as C
import os
import subprocess

import numpy as np
import pytest

from conftest import assert_close_f16, f32

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
B, S, V, D, HID, L = 16, 160, 144, 256, 512, 8
PROMPT = 18          # positions 0..17 prefilled; position 18 is the first fed
STEPS = 32
BASE, BINS = 3, 128


def test_kv_decoder_main_llm_matches_oracle(tmp_path, orc):
    exe = os.path.join(ROOT, "evk_amd", "bin", "kv_decoder_tool")
    assert os.path.exists(exe), "evk_amd/bin/kv_decoder_tool is not built: run `python -m evk_amd.build`"
    print("running", exe, "dump", flush=True)
    r = subprocess.run([exe, "dump", str(tmp_path), str(STEPS)], capture_output=True, text=True, timeout=110)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]

    cfg = orc.model_cfg(vocab=V, d=D, heads=1, layers=L, hidden=HID, max_seq=S)
    w = np.fromfile(tmp_path / "weights.bin", np.uint16)
    assert w.size == orc.lib().orc_model_weight_elems(C.byref(cfg))
    prompt = np.fromfile(tmp_path / "prompt.bin", np.uint16).reshape(B, PROMPT + 1)
    logits = np.fromfile(tmp_path / "logits.bin", np.uint16).reshape(STEPS, B, V)
    ids = np.fromfile(tmp_path / "ids.bin", np.uint16).reshape(STEPS, B)
    assert ((ids >= BASE) & (ids < BASE + BINS)).all()

    ties = 0
    worst = 0.0
    for b in range(B):
        cache = np.zeros(orc.lib().orc_model_cache_elems(C.byref(cfg)), np.uint16)
        for pos in range(PROMPT + 1):   # the logits of position 18 come with its token
            _, lg = orc.model_step(cfg, w, cache, int(prompt[b, pos]), pos)
        for s in range(STEPS):
            if s > 0:
                _, lg = orc.model_step(cfg, w, cache, int(ids[s - 1, b]), PROMPT + s)
            assert_close_f16(logits[s, b], lg, what=f"logits seq {b} step {s}")
            worst = max(worst, float(np.abs(f32(logits[s, b]) - f32(lg)).max()))
            sub = f32(lg)[BASE:BASE + BINS]
            want = BASE + int(np.argmax(sub))
            got = int(ids[s, b])
            if got != want:
                gap = abs(float(sub[got - BASE]) - float(sub[want - BASE]))
                assert gap < 1e-3, f"seq {b} step {s}: id {got} vs oracle {want} (gap {gap:.3g})"
                ties += 1
    print(f"{STEPS} steps x {B} sequences: max |dlogit| {worst:.4g}, {ties} near-ties", flush=True)
