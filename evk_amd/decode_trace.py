"""Stage timeline of the persistent decode (decode_persist) at BASELINE
configs[3], from the trace build of the library.

    python -m evk_amd.build --decode-trace      # evk_amd/_trace/libevkhip.so
    python evk_amd/decode_trace.py              # on the GPU

Runs the C4 model's 1024-token prefill, then 8 greedy steps at positions
1024..1031 in one persistent launch, and prints, for step 3 and layer 2, per
stage (S1 rms_norm+QKV+rope, S2 attention splits, S3 split merge+Wo+residual,
S4 rms_norm+W1+gelu, S5 W2+residual): how many workgroups take part, when
they start, when their input has arrived and when their outputs are stored
(100 MHz wall clock, microseconds from the layer's first start), and per
workgroup the wait for the input and the time from input to stored output;
then the hand-over into the layer, from layer 1's last S5 store.
"""
import ctypes as C
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
TRACE_LIB = os.path.join(HERE, "_trace", "libevkhip.so")


def main():
    if not os.path.exists(TRACE_LIB):
        sys.exit("evk_amd/_trace/libevkhip.so is missing: run `python -m evk_amd.build --decode-trace`")
    os.environ["EVKHIP_LIBRARY"] = TRACE_LIB
    sys.path.insert(0, ROOT)
    import numpy as np
    import torch

    import evk_amd as evk
    import oracle as orc

    dev = torch.device("cuda:0")
    evk.initialize()
    cfg, ocfg = evk.model_cfg(), orc.model_cfg()

    def to_dev(x):
        return torch.from_numpy(np.ascontiguousarray(x).view(np.int16)).view(torch.float16).to(dev)

    w = to_dev(orc.model_weights(ocfg, seed=301, std=0.02))
    prompt = torch.from_numpy(orc.tokens_u16(1024, 302, 32000).view(np.int16)).to(dev)
    cache = torch.zeros(evk.model_cache_elems(cfg), dtype=torch.float16, device=dev)
    tok = torch.zeros(9, dtype=torch.int16, device=dev)
    logits = torch.empty(cfg.vocab, dtype=torch.float16, device=dev)
    evk.model_prefill(cfg, w, cache, prompt, 0, tok, logits)
    packed = torch.empty(evk.model_packed_elems(cfg), dtype=torch.float16, device=dev)
    evk.model_pack(cfg, w, packed)
    first = tok[0].clone()
    ms = []
    for _ in range(4):  # the last launch's trace is read
        tok[0] = first
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        s.record()
        evk.model_decode_packed(cfg, packed, cache, tok, 8, 1024, logits)
        e.record()
        torch.cuda.synchronize()
        ms.append(s.elapsed_time(e))
    assert evk.device_status(clear=True) == 0, "the persistent decode reported a wait timeout"
    L = evk.lib()
    L.evkhip_debug_decode_trace.argtypes = [C.c_void_p]
    buf = np.zeros((2, 1024, 5, 3), np.uint64)
    assert L.evkhip_debug_decode_trace(buf.ctypes.data) == 0
    tt = buf.astype(np.int64)
    t, tprev = tt[1], tt[0]  # layer 2, layer 1
    took = t[:, :, 0] > 0
    t0 = t[:, 0, 0][took[:, 0]].min()
    us = (t - t0) * 0.01  # 100 MHz ticks -> us
    us_prev = (tprev - t0) * 0.01
    names = ["S1 rms_norm+QKV+rope", "S2 attention splits", "S3 merge+Wo+residual", "S4 rms_norm+W1+gelu",
             "S5 W2+residual"]
    print(f"# persistent decode stage timeline, C4 model (12 layers, d=768), step 3 of 8 (position 1027), layer 2")
    print(f"# launch of 8 steps: {min(ms):.3f} ms (best of {len(ms)}) = {min(ms) / 8 * 1000:.1f} us per step, "
          f"{min(ms) / 8 / 12 * 1000:.2f} us per layer on average (the LM head included)")
    print("# times in us from the layer's first S1 start (100 MHz wall clock, 0.01 us ticks); med/max over the "
          "workgroups of a stage")
    print(f"{'stage':24s} {'wgs':>4s} {'start med':>10s} {'input med':>10s} {'input max':>10s} {'done med':>9s} "
          f"{'done max':>9s} {'wait med':>9s} {'work med':>9s} {'work max':>9s}")
    for k in range(5):
        sel = took[:, k]
        if not sel.any():
            continue
        a, b, c = us[sel, k, 0], us[sel, k, 1], us[sel, k, 2]
        med = lambda x: float(np.median(x))
        print(f"{names[k]:24s} {int(sel.sum()):4d} {med(a):10.2f} {med(b):10.2f} {b.max():10.2f} {med(c):9.2f} "
              f"{c.max():9.2f} {med(b - a):9.2f} {med(c - b):9.2f} {(c - b).max():9.2f}")
    last = us[took[:, 4], 4, 2].max()
    print(f"# layer span (first S1 start to last S5 store): {last:.2f} us")
    took_prev = tprev[:, 4, 0] > 0
    if took_prev.any():
        prev_done = us_prev[took_prev, 4, 2].max()
        s1_in = float(np.median(us[took[:, 0], 0, 1]))
        print(f"# hop into the layer: layer 1's last S5 store at {prev_done:.2f} us, layer 2's S1 input (median) "
              f"at {s1_in:.2f} us: {s1_in - prev_done:.2f} us")
        # the chain from layer 1's last S5 store to layer 2's: per stage the hand-over (the producers' last
        # store to the consumers' median input) and the work (median input to the last store)
        hops, work, done = [], [], prev_done
        for k in range(5):
            sel = took[:, k]
            inp = float(np.median(us[sel, k, 1]))
            hops.append(inp - done)
            done = us[sel, k, 2].max()
            work.append(done - inp)
        print(f"# layer 2 from layer 1's last S5 store: {done - prev_done:.2f} us = hand-overs "
              f"{' + '.join(f'{h:.2f}' for h in hops)} = {sum(hops):.2f} us, stage work "
              f"{' + '.join(f'{w:.2f}' for w in work)} = {sum(work):.2f} us")


if __name__ == "__main__":
    main()
