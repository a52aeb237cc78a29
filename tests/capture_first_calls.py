"""Run by tests/test_gpu_capture.py in a fresh process: the library's first GEMV and GEMM calls
are made under stream capture (after tlx_attach_workspace, the only set-up call), then the graph
is replayed several times with eager work and synchronizations between the replays, and every
replay is compared bit for bit with the same calls made eagerly.  Prints one line per check and
exits 0 when all agree."""
import os
import sys

import numpy as np
import torch

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

from thunderllamax_amd import formats, ops, synth  # noqa: E402
from thunderllamax_amd._lib import LAYOUT_RAW, LAYOUT_TILED  # noqa: E402


def main():
    dev = torch.device("cuda:0")
    print("[capture] attach", flush=True)
    ops.attach_workspace(dev)
    rng = np.random.default_rng(31)
    g = formats.gridf_tensor(dev)
    # tiled ffn8 (shared partial tiles + counters), M = 11
    N, K, M = 2176, 5120, 11
    t = []
    for _ in range(2):
        p = torch.from_numpy(formats.iq3_pack_rows(synth.iq3xxs_raw(rng, N, K), K)).to(dev)
        tt = torch.empty(-(-N // 16) * 16 * 102 * (K // 256), dtype=torch.uint8, device=dev)
        ops.pack_iq3_tiled(p, tt, N, K)
        t.append(tt)
    x = torch.from_numpy(synth.activations_f16(rng, M, K)).to(dev)
    # prefill GEMM with split tiles (34 tiles: fewer than one round, split into k-segments)
    Mp, Np, Kp = 512, 2176, 1024
    p7 = [torch.from_numpy(formats.iq3_pack7(formats.iq3_pack_rows(synth.iq3xxs_raw(rng, Np, Kp), Kp), Kp)).to(dev)
          for _ in range(2)]
    xp = torch.from_numpy(synth.activations_f16(rng, Mp, Kp)).to(dev)
    # Q6_K GEMV (the k-quant kernels' one-time attribute)
    Nq = 4096
    wq = torch.from_numpy(synth.q6k_raw(rng, Nq, K)).to(dev)
    torch.cuda.synchronize()

    outs = [torch.empty(M, N, dtype=torch.float16, device=dev),
            torch.empty(Mp, Np, dtype=torch.float16, device=dev),
            torch.empty(M, Nq, dtype=torch.float16, device=dev)]

    def calls(o, s):
        ops.ffn8(t[0], t[1], g, x, o[0], layout=LAYOUT_TILED, stream=s)
        ops.pfg3_ffn(p7[0], p7[1], g, xp, o[1], stream=s)
        ops.q6k_gemv16(wq, x, o[2], LAYOUT_RAW, stream=s)

    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    print("[capture] first calls under capture", flush=True)
    with torch.cuda.graph(graph, stream=st):
        calls(outs, st)
    torch.cuda.synchronize()
    ref = [torch.empty_like(o) for o in outs]
    calls(ref, torch.cuda.current_stream())
    torch.cuda.synchronize()
    ok = True
    for rep in range(4):
        for o in outs:
            o.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        same = [torch.equal(a.view(torch.int16), b.view(torch.int16)) for a, b in zip(outs, ref)]
        print(f"[capture] replay {rep}: ffn8 {same[0]} pfg3_ffn {same[1]} q6k {same[2]}", flush=True)
        ok &= all(same)
        calls(ref, torch.cuda.current_stream())   # eager work between the replays
        torch.cuda.synchronize()
    print("[capture] OK" if ok else "[capture] MISMATCH", flush=True)
    return 0 if ok else 1


if __name__ == "__main__":
    sys.exit(main())
