"""Benchmark of the quantized-weight GEMV hot path on one MI355X.

Workload (``config.workload``): the IQ3_XXS fused FFN gate+up + SwiGLU GEMV of the dense
model, K=5120, N=2x17408 (68,239,360 weight bytes), at the speculative-verify widths
M in {1, 4, 8, 11}.  ``value`` is the achieved HBM throughput at M=11 in GB/s of algorithmic
bytes (weights + activations in + outputs out, counted once per call); the other widths are
reported under ``per_m``.  A "step" is one ffn8 call over one batch of M activation rows.

Timing: weights are synthetic (seeded) and resident in HBM before timing starts; each step
reads a different copy out of a rotation larger than the 256 MB Infinity Cache, so the
figure is HBM bandwidth, not cache bandwidth.  W untimed warmup steps, then K timed steps
(at least 20) captured in one HIP graph, as a decode step replays its launches, and the graph
replayed 5 times, each replay bracketed by device synchronization and timed with HIP events
recorded on the stream the graph replays on; ``ms_per_step`` is the median replay / K.
``roofline.traffic`` (and every leg's) is the HBM bytes per launch measured by rocprofv3
counters (the ``TRAFFIC`` table below, with the command that measured it).
The headline layout (``--layout``, default ``tiled``) is the library's tiled records (the GGUF
blocks re-encoded with precomputed table indices, 102 B per 256 weights, repacked on the GPU);
``value`` still counts the GGUF bytes (98 per 256 weights), so it is the rate at which the
quantized model streams.  ``per_m_other_layout`` times the reference's packed rows (pack_w1c),
where from M=6 on a step is two launches (the tile-ordered activation copy, then the GEMV), and
``per_m_pack7`` the packed7 units (/root/reference/engine/pack_w7.py), the plane the prefill GEMM
reads, on which the decode GEMVs run too (the reference's PF_DR7 mode).

Every figure (every leg) is the median of 5 graph replays, each of >= 20 calls and timed by its own
HIP events, after >= 3 eager warm-up calls and one untimed replay (``timing``).

``cpu_baseline`` times the numpy restatement of the reference's CPU path (dequantize, then
an fp32 matmul) on the same workload (config 2 at the headline M, timed in full: dequant and
matmul separately, median of 5 after one warm-up) on this host's cores; ``cpu`` holds the same
for every configuration (configs 3-5 on row / M slices, extrapolated linearly and labelled so).

``config1`` is BASELINE config 1: the Q6_K 5120x5120 GEMV with fp32 activations and outputs
(h6k2048's contract), weights rotated over more than 300 MB, graph replays, HBM roofline.
``stream`` is the measured HBM ceiling: a read-only stream over 1 GiB buffers (rotated), the
figure every GB/s roofline also states its fraction of (``frac_of_measured``) beside the 8 TB/s
datasheet peak (``frac``).

``gemm`` is the metric's second half: the prefill dequant-GEMM of config 4 at M=2048 and M=8192 --
gate+up with SwiGLU (K=5120, N=2x17408) and down with the residual epilogue (K=17408,
N=5120) -- in TFLOP/s (2*M*N*K per GEMM) and as a fraction of the dense fp16 MFMA peak;
``gemm.w4a8_ffn`` is the reference's int8-activation branch of the same gate+up (activation
quantizer + W4A8 GEMM), in TOP/s against the dense int8 MFMA peak.

``sweep`` is config 3: one dense hybrid decode step at M=11 -- 48 gated-delta-net layers and 16
attention layers (every fourth layer; Q6_K q on layers 3, 7, 19, 31, 43, 55, 59, 63) with their
FFNs, then the Q6_K head -- as the sequence of GEMV launches a decode step makes (10.18 GB of
weights, all resident, so every step streams them from HBM), captured once in a HIP graph and
replayed.  Weights are seeded random bytes with sane d fields (the timing does not depend on the
values; parity is the tests' business).  Reported as weight-streaming GB/s for the step.

``producers`` times the residual-add + RMSNorm producer in front of ffn8 at M=11, alone, then
followed by ffn8, and fused with it in one entry point (graph replays).

``formats`` times the load-time repacking on the GPU (raw GGUF IQ3_XXS rows of config 2's gate
matrix -> packed rows -> packed7) in GB/s of bytes read + written.

``moe`` is config 5: the whole MoE layer at M=11 and M=2048 as ``ops.moe_layer`` runs it by
default -- M=11: top-8 from N(0,1) logits, the pair-walk IQ4_XS gate+up and down (no sort)
with the shared expert's chunks in the same two launches, combine, all on one stream; M=2048: top-8, sort, grouped gate+up and down with
the shared expert's workgroups in the same two launches, combine -- seeded expert weights, the layer's launches per
step captured in one HIP graph (``ms_other_shared_stream``: the shared expert on the other
choice of stream; ``ms_sorted_grouped`` at M=11: the grouped route); each step reads a
different copy of the 257 expert slabs (3 copies, 1.3 GB), so at M=11 the weights come from
HBM.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

PEAK_HBM_GBS = 8000.0
# HBM bytes per launch (roofline.traffic), measured with two `rocprofv3 --pmc` passes over one
# command, FETCH_SIZE then WRITE_SIZE (KiB per dispatch, medians over each workload's dispatches):
#   bench.py --ms 11 --gemm-m 2048,8192 --no-sweep --no-formats --no-cpu --no-stream --steps 20
#            --warmup 3 --copy-mib 256
# and for the decode step `bench.py --sweep-only --steps 20 --warmup 3` (FETCH_SIZE and WRITE_SIZE
# summed over the 273 dispatches of one step, median over steps).  The 256 MiB device copy that ends
# the first command reads FETCH_SIZE = 131,094 KiB and WRITE_SIZE = 262,144 KiB, so fetched bytes =
# 2 x FETCH_SIZE x 1024 and written bytes = WRITE_SIZE x 1024.  Kernel + its helper launches (the
# tile-ordered activation copy of the packed-row GEMVs, the prefill GEMM's split-tile fix-up, the
# int8 quantizer, the MoE layer's router / sort / combine).  Re-measure when a kernel changes.
TRAFFIC = {
    "ffn8_m11_tiled": 75_370_291,       # iq3s_kernel<2,1,8,3>: F 35,840.9  W 1,922.0
    "ffn8_m11_packed": 74_799_514,      # iq3_xt_kernel + iq3_gemv_kernel<2,1,4,0>: F 65.0 + 36,191.2  W 160 + 374
    "ffn8_m11_pack7": 91_283_251,       # iq3_xt_kernel + iq3_gemv_kernel<2,1,4,1>: F 65.0 + 44,239.9  W 160 + 374
    "config1": 21_917_696,              # q6k_gemv_f32_kernel<5>: F 10,682.0  W 40.0
    "gemm_ffn_m2048": 992_334_848,      # pf_gemm<FFN> + pf_fix: F 384,159.0 + 32,795.5  W 131,072 + 4,096
    "gemm_down_m2048": 836_998_349,     # pf_gemm<RES> + pf_fix: F 244,813.4 + 81,948.0  W 122,880 + 40,978.4
    "gemm_ffn_m8192": 3_557_484_339,    # pf_gemm<FFN> (no split tiles): F 1,597,788.9  W 278,528
    "gemm_down_m8192": 1_753_614_131,   # pf_gemm<RES> + pf_fix: F 692,386.6 + 49,180.0  W 196,611.9 + 32,768.7
    "w4a8_ffn_m2048": 1_595_100_365,    # p8_quant + p8w4_ffn: F 10,256 + 728,025.6  W 11,520 + 69,632
    "merged_attnqkv_i3": 398_648_115,   # pfm_gemm_kernel: F 165,980.4  W 57,344
    "merged_attnqkv_q6": 652_394_086,   # pfm_gemm_kernel: F 289,879.8  W 57,344
    "merged_gdnqg": 542_371_430,        # pfm_gemm_kernel: F 232,061.8  W 65,536
    "moe_m11": 153_883_750,             # topk + pair-walk gate+up and down (shared inside) + combine: F 74,775.3  W 726.5
    "moe_m2048": 863_987_917,           # topk, sort, grouped gate+up / down with the shared expert, combine: F 354,038.1  W 135,662.0
    "ckpt_m11": 161_757_081,            # checkpoint classes, tiled slabs: topk, pair-walk IQ3_S up / Q6_K down with the Q8_0 shared expert inside, combine: F 78,619.7  W 726.5
    "ckpt_m2048": 939_681_894,          # checkpoint classes, tiled slabs: topk, sort, sorted up with the shared expert, register-decode down, shared down, combine: F 371,734.4  W 174,189.3
    "sweep": 12_030_388_122,            # one decode step: F 5,591,363.3  W 565,699.3
}
PEAK_F16_TFLOPS = 2500.0
PEAK_I8_TOPS = 5000.0
ROT_BYTES = 300 * 2**20
MEASURED = {"hbm_gbs": None}   # the read-stream ceiling of this run (stream leg), once measured


def hbm_roofline(achieved_gbs, kernel, traffic=None, **extra):
    """Roofline object of an HBM-bound measurement: fraction of the datasheet peak and, when the
    stream leg has run, of the measured read ceiling."""
    r = {"bound": "hbm", "achieved": round(achieved_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
         "frac": round(achieved_gbs / PEAK_HBM_GBS, 4), "traffic": traffic, "kernel": kernel}
    if MEASURED["hbm_gbs"]:
        r["measured_peak"] = MEASURED["hbm_gbs"]
        r["frac_of_measured"] = round(achieved_gbs / MEASURED["hbm_gbs"], 4)
    r.update(extra)
    return r


def mfma_roofline(achieved, kernel, peak=None, unit="TFLOP/s", traffic=None, **extra):
    peak = PEAK_F16_TFLOPS if peak is None else peak
    r = {"bound": "mfma", "achieved": round(achieved, 1), "peak": peak, "unit": unit,
         "frac": round(achieved / peak, 4), "traffic": traffic, "kernel": kernel}
    r.update(extra)
    return r


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-formats", action="store_true", help="skip the producer and load-time repacking legs")
    ap.add_argument("--ms", default="1,4,8,11", help="activation widths to time")
    ap.add_argument("--gemm-m", default="2048,8192", help="prefill row counts for the GEMM leg ('0': skip)")
    ap.add_argument("--no-config1", action="store_true", help="skip the config-1 Q6_K fp32 GEMV leg")
    ap.add_argument("--no-stream", action="store_true", help="skip the HBM read-stream ceiling leg")
    ap.add_argument("--cpu-reps", type=int, default=5, help="timed repetitions of each CPU baseline (median)")
    ap.add_argument("--no-moe", action="store_true", help="skip the MoE leg")
    ap.add_argument("--no-sweep", action="store_true", help="skip the decode-step sweep leg")
    ap.add_argument("--sweep-only", action="store_true",
                    help="run only the decode-step sweep (no per-layer-kind graphs) and print its object: "
                         "the form a counter pass over one step's dispatches uses")
    ap.add_argument("--layout", default="tiled", choices=("tiled", "packed"),
                    help="IQ3_XXS weight layout of the headline ffn8 leg (the other one is "
                         "reported under per_m_other_layout)")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="end with one device-to-device copy of this many MiB (a reference "
                         "dispatch of known size for calibrating memory counters)")
    return ap.parse_args()


# Every timed figure: a HIP graph of `calls` (>= MIN_CALLS) calls -- each may read a different
# rotated weight copy -- captured after >= MIN_WARM eager warm-up calls and replayed once untimed;
# then NREP replays, each bracketed by its own HIP events on the replay stream; the figure is the
# median over those replays of (replay time / calls).
MIN_CALLS, MIN_WARM, NREP = 20, 3, 5
TIMING = (f"median of {NREP} graph replays of >= {MIN_CALLS} calls each (HIP events around each replay), "
          f"after >= {MIN_WARM} eager warm-up calls and one untimed replay")


def _timed_replays(g, calls, torch):
    ts = []
    for _ in range(NREP):
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record()
        g.replay()   # replays on the current stream
        t1.record()
        torch.cuda.synchronize()
        ts.append(t0.elapsed_time(t1) / calls)
    return float(np.median(ts))


def time_graph(fn, steps, warmup, torch):
    """Median ms of fn(stream) per call (see TIMING): max(steps, MIN_CALLS) calls captured in one
    HIP graph (host launch gaps excluded: a decode step replays its launches as a graph; each call
    may pick different buffers, e.g. rotated weights), after max(warmup, MIN_WARM) eager calls --
    the one-time set-up happens outside the capture."""
    calls = max(steps, MIN_CALLS)
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        for _ in range(max(warmup, MIN_WARM)):
            fn(st)
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        for _ in range(calls):
            fn(st)
    g.replay()
    torch.cuda.synchronize()
    return _timed_replays(g, calls, torch)


def time_ffn(ops, wsets, gridf, x, gact, steps, warmup, torch, layout=1):
    """Median ms per ffn8 call (time_graph), each call on the next rotated weight copy."""
    n = len(wsets)
    it = [0]

    def call(st):
        wg, wu = wsets[it[0] % n]
        it[0] += 1
        ops.ffn8(wg, wu, gridf, x, gact, layout=layout, stream=st)

    return time_graph(call, steps, warmup, torch)


def time_call(fn, steps, warmup, torch):
    """Median ms of fn(stream) over NREP timings of max(steps, MIN_CALLS) eager calls each, after
    max(warmup, MIN_WARM) warm-up calls, HIP events on its stream."""
    stream = torch.cuda.current_stream()
    calls = max(steps, MIN_CALLS)
    for _ in range(max(warmup, MIN_WARM)):
        fn(stream)
    torch.cuda.synchronize()
    ts = []
    for _ in range(NREP):
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        for _ in range(calls):
            fn(stream)
        t1.record(stream)
        torch.cuda.synchronize()
        ts.append(t0.elapsed_time(t1) / calls)
    return float(np.median(ts))


def gemm_weights(formats, synth, torch, dev):
    """Config 4's weights in the packed7 unit layout the prefill GEMMs read (seeded)."""
    rng = synth.config_rng(4)
    H, F = 5120, 17408
    def pack7(rows, k):
        return torch.from_numpy(formats.iq3_pack7(formats.iq3_pack_rows(synth.iq3xxs_raw(rng, rows, k), k), k)).to(dev)
    return pack7(F, H), pack7(F, H), pack7(H, F)


def gemm_leg(ops, formats, synth, torch, dev, M, steps, warmup, weights, w4a8=True):
    """Config 4: IQ3_XXS FFN prefill GEMMs at M rows, synthetic seeded weights, graph replays."""
    rng = synth.config_rng(4)
    H, F = 5120, 17408
    pg, pu, pd = weights
    gridf = formats.gridf_tensor(dev)
    x = torch.from_numpy(synth.activations_f16(rng, M, H)).to(dev)
    act = torch.empty(M, F, dtype=torch.float16, device=dev)
    res = torch.randn(M, H, device=dev)
    y = torch.empty(M, H, dtype=torch.float32, device=dev)
    t_ffn = time_graph(lambda s: ops.pfg3_ffn(pg, pu, gridf, x, act, stream=s), steps, warmup, torch)
    t_down = time_graph(lambda s: ops.pfg3_iq3d(pd, gridf, act, res, y, stream=s), steps, warmup, torch)
    f_ffn, f_down = 2.0 * M * H * 2 * F, 2.0 * M * F * H
    tf_ffn = f_ffn / (t_ffn * 1e-3) / 1e12
    tf_down = f_down / (t_down * 1e-3) / 1e12
    tf_layer = (f_ffn + f_down) / ((t_ffn + t_down) * 1e-3) / 1e12
    out = {
        "workload": f"IQ3_XXS prefill FFN, M={M}: gate+up+SwiGLU K={H} N=2x{F}; down+residual K={F} N={H}",
        "M": M,
        "ffn_ms": round(t_ffn, 4), "ffn_tflops": round(tf_ffn, 1),
        "down_ms": round(t_down, 4), "down_tflops": round(tf_down, 1),
        "tflops": round(tf_layer, 1),
        "roofline": mfma_roofline(tf_ffn, "pf_gemm_kernel<FFN> (+ pf_fix_kernel) gate+up",
                                  traffic=TRAFFIC.get(f"gemm_ffn_m{M}"),
                                  down=mfma_roofline(tf_down, "pf_gemm_kernel<RES> (+ pf_fix_kernel) down",
                                                     traffic=TRAFFIC.get(f"gemm_down_m{M}"))),
    }
    if not w4a8:
        return out
    # the int8-activation branch of the same FFN: quantize the activations, then the W4A8 GEMM
    xq = torch.empty(M, H, dtype=torch.int8, device=dev)
    sx = torch.empty(M, H // 128, dtype=torch.float32, device=dev)
    rs = torch.empty(M, H // 128, dtype=torch.int32, device=dev)
    lut8 = formats.lut8_tensor(dev)
    t_q8 = time_graph(lambda s: ops.p8_quant(x, xq, sx, rs, stream=s), steps, warmup, torch)
    t_w4 = time_graph(lambda s: ops.p8w4_ffn(pg, pu, lut8, xq, sx, act, stream=s), steps, warmup, torch)
    to_w4 = f_ffn / ((t_q8 + t_w4) * 1e-3) / 1e12
    out["w4a8_ffn"] = {"quant_ms": round(t_q8, 4), "gemm_ms": round(t_w4, 4), "tops": round(to_w4, 1),
                       "roofline": mfma_roofline(to_w4, "p8_quant_kernel + p8w4_ffn_kernel", PEAK_I8_TOPS, "TOP/s",
                                                 traffic=TRAFFIC.get(f"w4a8_ffn_m{M}"))}
    return out


def merged_gemm_leg(ops, formats, synth, torch, dev, M, steps, warmup):
    """The merged multi-class prefill GEMM (pf_gemm3m) at M rows, K=5120, on the reference's three
    configurations (/root/reference/engine/build_p7b.py:58-77): attention q/k/v with an IQ3_XXS or a
    Q6_K q (IQ3_XXS k, Q4_K v) and the GDN qkv (Q5_K) with its IQ3_XXS gate.  Seeded weights, graph
    replays, TFLOP/s of 2*M*N*K summed over the segments."""
    from thunderllamax_amd._lib import (LAYOUT_PACK7, LAYOUT_PACKED, LAYOUT_RAW, TYPE_IQ3_XXS, TYPE_Q4_K,
                                        TYPE_Q5_K, TYPE_Q6_K)
    K = 5120
    rng = synth.config_rng(4)

    def mat(cls, n):
        if cls == "iq3":
            a = formats.iq3_pack7(formats.iq3_pack_rows(synth.iq3xxs_raw(rng, n, K), K), K)
            t, lay = TYPE_IQ3_XXS, LAYOUT_PACK7
        elif cls == "q6k":
            a, t, lay = formats.q6_pad_rows(synth.q6k_raw(rng, n, K), K), TYPE_Q6_K, LAYOUT_PACKED
        else:
            a = synth.k4_raw(rng, n, K, cls == "q5k")
            t, lay = (TYPE_Q5_K if cls == "q5k" else TYPE_Q4_K), LAYOUT_RAW
        return torch.from_numpy(np.ascontiguousarray(a).reshape(-1)).to(dev), t, lay, n

    configs = {"attnqkv_i3": [("iq3", 12288), ("iq3", 1024), ("q4k", 1024)],
               "attnqkv_q6": [("q6k", 12288), ("iq3", 1024), ("q4k", 1024)],
               "gdnqg": [("q5k", 10240), ("iq3", 6144)]}
    gridf = formats.gridf_tensor(dev)
    x = torch.from_numpy(synth.activations_f16(rng, M, K)).to(dev)
    out = {"workload": f"merged prefill GEMM (pf_gemm3m), M={M}, K={K}: segments of different weight classes "
                       "sharing x, one launch, fp16 out"}
    for name, segs in configs.items():
        mats = [mat(c, n) for c, n in segs]
        outs = [torch.empty(M, n, dtype=torch.float16, device=dev) for *_, n in mats]
        t = time_graph(lambda s: ops.pfg3m([m[0] for m in mats], outs, [m[1] for m in mats], [m[2] for m in mats],
                                           gridf, x, stream=s), steps, warmup, torch)
        flops = 2.0 * M * K * sum(n for *_, n in mats)
        tf = flops / (t * 1e-3) / 1e12
        out[name] = {"segments": [f"{c} {n}x{K}" for c, n in segs], "ms": round(t, 4), "tflops": round(tf, 1),
                     "roofline": mfma_roofline(tf, "pfm_gemm_kernel (one launch over the segments)",
                                                  traffic=TRAFFIC.get(f"merged_{name}") if M == 2048 else None)}
        del mats, outs
    return out


def producers_leg(ops, formats, synth, torch, dev, steps, warmup, M=11, tiled=True):
    """The activation producer before the FFN GEMV (hh{M}: residual add + RMSNorm -> fp16) at
    config 2's D=5120, alone, followed by ffn8, and fused with it (tlx_ffn8_hh), as graph
    replays over rotated FFN weights (tiled records or packed rows)."""
    from thunderllamax_amd._lib import LAYOUT_PACKED, LAYOUT_TILED
    K, N = 5120, 17408
    rng = synth.config_rng(2)
    lay = LAYOUT_TILED if tiled else LAYOUT_PACKED

    def mat():
        w = torch.from_numpy(formats.iq3_pack_rows(synth.iq3xxs_raw(rng, N, K), K)).to(dev)
        if not tiled:
            return w
        t = torch.empty(N * 102 * (K // 256), dtype=torch.uint8, device=dev)
        ops.pack_iq3_tiled(w, t, N, K)
        return t

    copies = [(mat(), mat()) for _ in range(max(1, -(-ROT_BYTES // (2 * N * 98 * (K // 256)))))]
    gridf = formats.gridf_tensor(dev)
    x = torch.randn(M, K, device=dev)
    a = torch.randn(M, K, device=dev).half()
    nw = torch.ones(K, device=dev)
    hh = torch.empty(M, K, device=dev)
    hhx = torch.empty(M, K, dtype=torch.float16, device=dev)
    g = torch.empty(M, N, dtype=torch.float16, device=dev)
    it = [0]

    def pick():
        it[0] += 1
        return copies[it[0] % len(copies)]

    def sep(s):
        wg, wu = pick()
        ops.add_rms_f16(x, a, nw, hh, hhx, stream=s)
        ops.ffn8(wg, wu, gridf, hhx, g, layout=lay, stream=s)

    def fused(s):
        wg, wu = pick()
        ops.ffn8_hh(wg, wu, gridf, x, a, nw, hh, hhx, g, layout=lay, stream=s)

    t_norm = time_graph(lambda s: ops.add_rms_f16(x, a, nw, hh, hhx, stream=s), steps, warmup, torch)
    t_sep = time_graph(sep, steps, warmup, torch)
    t_fused = time_graph(fused, steps, warmup, torch)
    return {"workload": f"hh{{M}} producer (D={K}) + ffn8 (N=2x{N}), M={M}",
            "iq3_layout": "tiled records" if tiled else "packed rows",
            "add_rms_us": round(t_norm * 1e3, 2), "add_rms_then_ffn8_us": round(t_sep * 1e3, 2),
            "ffn8_hh_us": round(t_fused * 1e3, 2)}


def formats_leg(ops, synth, torch, dev, steps, warmup):
    """Load-time repacking of config 2's gate matrix on the GPU (raw GGUF rows -> packed rows
    -> packed7): HBM bytes moved (read + write) per second."""
    N, K = 17408, 5120
    raw = torch.from_numpy(synth.iq3xxs_raw(synth.config_rng(2), N, K).reshape(-1)).to(dev)
    packed = torch.empty_like(raw)
    p7 = torch.empty(N * K // 2, dtype=torch.uint8, device=dev)
    t_rows = time_call(lambda s: ops.pack_iq3_rows(raw, packed, N, K, stream=s), steps, warmup, torch)
    t_p7 = time_call(lambda s: ops.pack_w7(packed, p7, N, K, stream=s), steps, warmup, torch)
    nb = raw.numel()
    return {"workload": f"IQ3_XXS {N}x{K} ({nb} B): raw rows -> packed rows -> packed7",
            "pack_rows_ms": round(t_rows, 4), "pack_rows_gbs": round(2 * nb / (t_rows * 1e-3) / 1e9, 1),
            "pack_w7_ms": round(t_p7, 4), "pack_w7_gbs": round((nb + p7.numel()) / (t_p7 * 1e-3) / 1e9, 1)}


def moe_leg(ops, formats, synth, torch, dev, steps, warmup):
    """Config 5: the MoE layer at M=11 (HBM-bound) and M=2048 (MFMA-bound)."""
    from thunderllamax_amd._lib import LAYOUT_RAW, LAYOUT_TILED
    rng = synth.config_rng(5)
    E, H, F = 256, 2048, 512
    copies = {LAYOUT_RAW: [], LAYOUT_TILED: []}   # GGUF rows, and the same slabs repacked as tiled records

    def tables(dgu, ddn):
        return dict(keep=(dgu, ddn), ptbl=formats.pointer_table(dgu[:E], dev),
                    ptbl_dn=formats.pointer_table(ddn[:E], dev), ptbl_sh=formats.pointer_table([dgu[E], ddn[E]], dev))

    for _ in range(3):
        gu, dn = synth.moe_expert_slabs(rng, E + 1)
        dgu = [torch.from_numpy(a).to(dev) for a in gu]
        ddn = [torch.from_numpy(a).to(dev) for a in dn]
        copies[LAYOUT_RAW].append(tables(dgu, ddn))
        copies[LAYOUT_TILED].append(tables([ops.pack_iq4_tiled(a, torch.empty_like(a), 2 * F, H) for a in dgu],
                                           [ops.pack_iq4_tiled(a, torch.empty_like(a), H, F) for a in ddn]))
    iq4nl = formats.iq4nl_tensor(dev)
    out = {"workload": "MoE layer, 256 IQ4_XS experts + 1 shared, hidden 2048, FF 512, top-8; hidden states "
                       "bf16(0.05 * N(0,1)) (N(0,1) overflows the fp16 parts for these weight statistics); "
                       "expert slabs as tiled records (tlx_pack_iq4_tiled, the GGUF bytes permuted into lane order)"}
    for P in (11, 2048):
        np_ = 8 * P
        x = torch.from_numpy(synth.bf16_round(0.05 * rng.standard_normal((P, H)).astype(np.float32))).to(dev)
        logits = torch.from_numpy(rng.standard_normal((P, E)).astype(np.float32)).to(dev)
        sg = torch.rand(P, device=dev)
        hres = torch.randn(P, H, device=dev)
        sc = ops.MoeScratch(P, dev)
        y = torch.empty(P, H, device=dev)
        state = {"i": 0}

        def layer(st, overlap=None, layout=LAYOUT_TILED, pair_walk=None):
            c = copies[layout][state["i"] % 3]
            state["i"] += 1
            ops.moe_layer(logits, sg, x, hres, y, c["ptbl"], c["ptbl_dn"], c["ptbl_sh"], iq4nl, sc, stream=st,
                          overlap_shared=overlap, layout=layout, pair_walk=pair_walk)

        walk = P <= ops.MOE_PAIR_WALK_MAX_P   # the layer's defaults: the shared expert in the routed launches
        t_other = time_graph(lambda st: layer(st, True), steps, warmup, torch)
        t_raw = time_graph(lambda st: layer(st, None, LAYOUT_RAW), steps, warmup, torch)
        t_grouped = time_graph(lambda st: layer(st, False, pair_walk=False), steps, warmup, torch) if walk else None
        t = time_graph(lambda st: layer(st), steps, warmup, torch)
        hit = int(torch.unique(sc.eids).numel())
        flops = 2.0 * 3 * F * H * (8 * P + P)
        wbytes = (hit + 1) * 1671168
        tflops = flops / (t * 1e-3) / 1e12
        gbs = wbytes / (t * 1e-3) / 1e9
        route = ("top-8, pair walk (no sort) with the shared expert in its two launches" if walk else
                 "top-8, sort, grouped expert GEMMs with the shared expert in their two launches")
        out[f"M{P}"] = {"ms": round(t, 4), "tflops": round(tflops, 2), "route": route,
                        "experts_hit": hit, "weight_gbs": round(gbs, 1),
                        "ms_other_shared_stream": round(t_other, 4), "ms_gguf_row_slabs": round(t_raw, 4),
                        **({"ms_sorted_grouped": round(t_grouped, 4)} if walk else {}),
                        "roofline": (hbm_roofline(gbs, f"MoE layer ({route}, combine; graph): "
                                                       "expert weight bytes / layer time",
                                                  traffic=TRAFFIC.get(f"moe_m{P}"))
                                     if P <= 64 else
                                     mfma_roofline(tflops, f"MoE layer ({route}, combine; graph): "
                                                           "2*3*512*2048*9*M / layer time",
                                                   traffic=TRAFFIC.get(f"moe_m{P}")))}
    return out


def moe_ckpt_leg(ops, formats, synth, torch, dev, steps, warmup):
    """The MoE layer with the reference checkpoint's weight classes (IQ3_S routed gate/up, Q6_K
    routed down, Q8_0 shared expert; ops.moe_layer_ckpt) at M=11 and M=2048, config 5's shapes,
    seeded weights (a synthetic IQ3_S grid), two copies of the slabs rotated (906 MB), graph
    replays; FLOPs and expert bytes counted as for config 5.  The routed slabs are timed as tiled
    records (tlx_pack_iq3s_tiled / tlx_pack_q6k_tiled, the layout's headline) and as GGUF rows."""
    from thunderllamax_amd._lib import LAYOUT_RAW, LAYOUT_TILED
    rng = np.random.default_rng(20261205)
    E, H, F = 256, 2048, 512
    sets = {LAYOUT_RAW: [], LAYOUT_TILED: []}
    for _ in range(2):
        gu, dn, shared = synth.moe_ckpt_slabs(rng, E)
        dgu = [torch.from_numpy(a).to(dev) for a in gu]
        ddn = [torch.from_numpy(a).to(dev) for a in dn]
        sh = [torch.from_numpy(np.ascontiguousarray(a).reshape(-1)).to(dev) for a in shared]
        tgu = [ops.pack_iq3s_tiled(a, torch.empty_like(a), 2 * F, H) for a in dgu]
        tdn = [ops.pack_q6k_tiled(a, torch.empty_like(a), H, F) for a in ddn]
        sets[LAYOUT_RAW].append(dict(keep=(dgu, ddn), ptbl=formats.pointer_table(dgu, dev),
                                     ptbl_dn=formats.pointer_table(ddn, dev), sh=sh))
        sets[LAYOUT_TILED].append(dict(keep=(tgu, tdn), ptbl=formats.pointer_table(tgu, dev),
                                       ptbl_dn=formats.pointer_table(tdn, dev), sh=sh))
    gridf = torch.from_numpy(synth.iq3s_grid(rng).reshape(-1)).to(dev)
    out = {"workload": "MoE layer with the checkpoint's classes: 256 IQ3_S gate/up + Q6_K down experts, Q8_0 shared "
                       "expert, hidden 2048, FF 512, top-8; hidden states bf16(0.05 * N(0,1))"}
    for P in (11, 2048):
        x = torch.from_numpy(synth.bf16_round(0.05 * rng.standard_normal((P, H)).astype(np.float32))).to(dev)
        logits = torch.from_numpy(rng.standard_normal((P, E)).astype(np.float32)).to(dev)
        sg = torch.rand(P, device=dev)
        hres = torch.randn(P, H, device=dev)
        sc = ops.MoeScratch(P, dev)
        y = torch.empty(P, H, device=dev)
        state = {"i": 0}

        def layer(st, layout=LAYOUT_TILED):
            c = sets[layout][state["i"] % 2]
            state["i"] += 1
            ops.moe_layer_ckpt(logits, sg, x, hres, y, c["ptbl"], c["ptbl_dn"], c["sh"], gridf, sc, stream=st,
                               layout=layout)

        t_rows = time_graph(lambda st: layer(st, LAYOUT_RAW), steps, warmup, torch)
        t = time_graph(layer, steps, warmup, torch)
        hit = int(torch.unique(sc.eids).numel())
        flops = 2.0 * 3 * F * H * (8 * P + P)
        wbytes = hit * (2 * F * 880 + H * 420) + 2 * F * 2176 + H * 544
        tflops = flops / (t * 1e-3) / 1e12
        gbs = wbytes / (t * 1e-3) / 1e9
        route = ("pair walk with the shared expert inside" if P <= ops.MOE_PAIR_WALK_MAX_P else
                 "sort + sorted forms with the shared expert inside")
        out[f"M{P}"] = {"ms": round(t, 4), "tflops": round(tflops, 2), "experts_hit": hit, "weight_gbs": round(gbs, 1),
                        "route": route, "slabs": "tiled records", "ms_gguf_rows": round(t_rows, 4),
                        "roofline": (hbm_roofline(gbs, f"checkpoint-class MoE layer ({route}; graph): expert bytes / "
                                                       "layer time", traffic=TRAFFIC.get(f"ckpt_m{P}")) if P <= 64 else
                                     mfma_roofline(tflops, f"checkpoint-class MoE layer ({route}; graph): "
                                                           "2*3*512*2048*9*M / layer time",
                                                   traffic=TRAFFIC.get(f"ckpt_m{P}")))}
    return out


def sweep_leg(ops, formats, torch, dev, steps, warmup, tiled=True, per_kind_graphs=True):
    """Config 3: the 64-layer dense decode step at M=11 plus the Q6_K head.  With ``tiled`` every
    IQ3_XXS tensor except the k/v rows beside a Q6_K q reads tiled records (repacked on the GPU
    from the packed rows).  The four GDN projections that read the same x share one launch, and
    each FFN block hands ffn8's output to down8 in the tile-ordered form (no activation copy)."""
    from thunderllamax_amd._lib import LAYOUT_PACKED, LAYOUT_RAW, LAYOUT_TILED
    lay = LAYOUT_TILED if tiled else LAYOUT_PACKED
    H, F, M = 5120, 17408, 11
    gen = torch.Generator(device=dev)
    gen.manual_seed(20261204)
    dbits = 0x1419  # fp16 1.05e-3: a finite scale for every block

    def iq3(rows, k):      # packed rows [qs 64NB][sw 32NB][d 2NB]
        nb = k // 256
        w = torch.randint(0, 256, (rows, 98 * nb), dtype=torch.uint8, device=dev, generator=gen)
        w[:, 96 * nb:].view(torch.int16).fill_(dbits)
        return w

    def iq3t(rows, k):     # the same, as tiled records when ``tiled``; bytes counted as GGUF
        w = iq3(rows, k)
        if not tiled:
            return w, w.numel()
        t = torch.empty((rows + 15) // 16 * 16 * 102 * (k // 256), dtype=torch.uint8, device=dev)
        ops.pack_iq3_tiled(w, t, rows, k)
        return t, w.numel()

    def q6(rows, k):       # GGUF 210-B blocks, d at bytes 208..209
        nb = k // 256
        w = torch.randint(0, 256, (rows, nb, 210), dtype=torch.uint8, device=dev, generator=gen)
        w[:, :, 208:210].view(torch.int16).fill_(dbits)
        return w.view(rows, nb * 210)

    gridf = formats.gridf_tensor(dev)
    xs = {k: torch.randn(M, k, device=dev).half() for k in (H, 6144, F)}
    o = {n: torch.empty(M, n, dtype=torch.float16, device=dev) for n in (10240, 6144, 48, 12288, 1024, H, F)}
    gt = ops.tileord_empty(F, dev)   # ffn8's output in the tile-ordered form (tiled records)
    vrow = torch.empty(M, 1024, dtype=torch.float16, device=dev)
    ab48 = torch.empty(M, 48, dtype=torch.float16, device=dev)
    hh = torch.randn(M, H, device=dev)
    y = torch.empty(M, H, device=dev)
    logits = torch.empty(M, 151936, dtype=torch.float16, device=dev)
    q6_layers = {3, 7, 19, 31, 43, 55, 59, 63}
    calls, nbytes = [], 0
    kinds = {"gdn": [], "attn_iq3": [], "attn_q6": [], "head": []}
    for layer in range(64):
        c0 = len(calls)
        if layer % 4 == 3:   # full attention
            wo, nbo = iq3t(H, 6144)
            if layer in q6_layers:
                wq, wk, wv = q6(12288, H), iq3(1024, H), iq3(1024, H)
                calls.append(lambda s, wq=wq, wk=wk, wv=wv: ops.aq6k8(wq, wk, wv, gridf, xs[H], o[12288], o[1024], vrow, layout=LAYOUT_RAW, stream=s))
                nbytes += wq.numel() + wk.numel() + wv.numel()
                kind = "attn_q6"
            else:
                (wq, nbq), (wk, nbk), (wv, nbv) = iq3t(12288, H), iq3t(1024, H), iq3t(1024, H)
                calls.append(lambda s, wq=wq, wk=wk, wv=wv: ops.aq3k8(wq, wk, wv, gridf, xs[H], o[12288], o[1024], vrow, layout=lay, stream=s))
                nbytes += nbq + nbk + nbv
                kind = "attn_iq3"
            calls.append(lambda s, w=wo: ops.iq3_gemv(w, gridf, xs[6144], o[H], layout=lay, stream=s))
            nbytes += nbo
        else:                # gated delta net projections
            # qkv, gate, alpha, beta read the same x: one launch (tlx_iq3_gemv_multi); then ssm_out
            proj = [iq3t(10240, H), iq3t(6144, H), iq3t(48, H), iq3t(48, H)]
            pw = [w for w, _ in proj]
            calls.append(lambda s, pw=pw: ops.iq3_gemv_multi(pw, gridf, xs[H], [o[10240], o[6144], o[48], ab48], layout=lay, stream=s))
            wso, nbso = iq3t(H, 6144)
            calls.append(lambda s, w=wso: ops.iq3_gemv(w, gridf, xs[6144], o[H], layout=lay, stream=s))
            nbytes += sum(nb for _, nb in proj) + nbso
            kind = "gdn"
        (wg, nbg), (wu, nbu), (wd, nbd) = iq3t(F, H), iq3t(F, H), iq3t(H, F)
        if tiled:   # the FFN block's hand-off: ffn8 writes the tile-ordered form down8 reads (no copy)
            calls.append(lambda s, wg=wg, wu=wu: ops.ffn8(wg, wu, gridf, xs[H], gt, layout=lay, stream=s,
                                                          out_tileord=True))
            calls.append(lambda s, wd=wd: ops.down8(wd, gridf, gt, hh, y, layout=lay, stream=s, in_tileord=True))
        else:
            calls.append(lambda s, wg=wg, wu=wu: ops.ffn8(wg, wu, gridf, xs[H], o[F], layout=lay, stream=s))
            calls.append(lambda s, wd=wd: ops.down8(wd, gridf, o[F], hh, y, layout=lay, stream=s))
        nbytes += nbg + nbu + nbd
        kinds[kind].append((c0, len(calls)))
    wh = q6(151936, H)
    c0 = len(calls)
    calls.append(lambda s: ops.q6k_gemv16(wh, xs[H], logits, LAYOUT_RAW, stream=s))
    kinds["head"].append((c0, len(calls)))
    nbytes += wh.numel()

    def graph_ms(lo, hi, reps, warm):
        """Median ms of one replay of calls[lo:hi] (each replay timed by its own events)."""
        st = torch.cuda.Stream()
        st.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(st):
            for _ in range(max(warm, MIN_WARM)):
                for c in calls[lo:hi]:
                    c(st)      # eager first: one-time kernel attributes are set outside capture
        torch.cuda.current_stream().wait_stream(st)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=st):
            for c in calls[lo:hi]:
                c(st)
        g.replay()
        torch.cuda.synchronize()
        ts = []
        for _ in range(max(reps, MIN_CALLS)):
            t0 = torch.cuda.Event(enable_timing=True)
            t1 = torch.cuda.Event(enable_timing=True)
            t0.record()
            g.replay()
            t1.record()
            torch.cuda.synchronize()
            ts.append(t0.elapsed_time(t1))
        return float(np.median(ts))

    t_step = graph_ms(0, len(calls), steps, warmup)
    per_kind = {}
    for kind, spans in (kinds.items() if per_kind_graphs else ()):   # one layer of each kind, replayed
        lo, hi = spans[0]
        t = graph_ms(lo, hi, steps, warmup)
        per_kind[kind] = {"layers": len(spans), "ms_per_layer": round(t, 4)}
    gbs = nbytes / (t_step * 1e-3) / 1e9
    return {"workload": "dense hybrid decode step, M=11: 48 GDN + 16 attention layers (8 with a Q6_K q), "
                        "FFN 17408, Q6_K head 151936x5120",
            "iq3_layout": "tiled records" if tiled else "packed rows",
            "M": M, "launches": len(calls), "weight_bytes": nbytes, "ms": round(t_step, 4),
            "weight_gbs": round(gbs, 1), "frac_of_peak": round(gbs / PEAK_HBM_GBS, 4),
            "per_layer_kind": per_kind,
            "roofline": hbm_roofline(gbs, f"decode step: {len(calls)} GEMV launches in one graph "
                                          "(weight bytes per step / step time)",
                                     traffic=TRAFFIC["sweep"] if tiled else None)}


def config1_leg(ops, synth, torch, dev, steps, warmup):
    """Config 1: Q6_K 5120x5120 GEMV, fp32 x and y (tlx_q6k_gemv, the h6k2048 contract), weights
    rotated over more than 300 MB so every step reads HBM."""
    from thunderllamax_amd._lib import LAYOUT_RAW
    rng = synth.config_rng(1)
    N = K = 5120
    wbytes = N * 210 * (K // 256)
    copies = [torch.from_numpy(synth.q6k_raw(rng, N, K)).to(dev) for _ in range(-(-ROT_BYTES // wbytes))]
    x = torch.from_numpy(rng.standard_normal(K).astype(np.float32)).to(dev)
    y = torch.empty(N, dtype=torch.float32, device=dev)
    it = [0]

    def step(s):
        it[0] += 1
        ops.h6k_gemv(copies[it[0] % len(copies)], x, y, layout=LAYOUT_RAW, stream=s)

    t = time_graph(step, steps, warmup, torch)
    nbytes = wbytes + 4 * K + 4 * N
    gbs = nbytes / (t * 1e-3) / 1e9
    return {"workload": f"Q6_K GEMV {N}x{K}, fp32 x and y (M=1), raw 210-B blocks", "ms": round(t, 5),
            "algorithmic_bytes": nbytes, "gbs": round(gbs, 1), "rotation_copies": len(copies),
            "roofline": hbm_roofline(gbs, "q6k_gemv_f32_kernel", traffic=TRAFFIC["config1"])}


def stream_leg(ops, torch, dev, steps, warmup):
    """Measured HBM read ceiling: tlx_stream_read over two 1 GiB buffers in turn (each step reads
    1 GiB; 2 GiB rotate past the 256 MB Infinity Cache)."""
    nbytes = 1 << 30
    bufs = [torch.ones(nbytes // 4, dtype=torch.int32, device=dev) for _ in range(2)]
    sink = torch.empty(4 * nbytes // ops.stream_chunk_bytes(), dtype=torch.int32, device=dev)
    it = [0]

    def step(s):
        it[0] += 1
        ops.stream_read(bufs[it[0] % 2], sink, stream=s)

    t = time_graph(step, steps, warmup, torch)
    gbs = nbytes / (t * 1e-3) / 1e9
    MEASURED["hbm_gbs"] = round(gbs, 1)
    return {"workload": "read-only stream, 1 GiB per step (2 buffers rotated), 16-B loads, 64 KB per workgroup",
            "ms": round(t, 4), "gbs": round(gbs, 1), "frac_of_datasheet": round(gbs / PEAK_HBM_GBS, 4),
            "kernel": "stream_read_kernel"}


# ------------------------------------------------------------------ CPU baselines
def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.lower().startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


class _Cpu:
    """Numpy restatement of the reference's CPU path (the oracle's dequantizers, then fp32
    matmuls): row chunks dequantized on a thread pool (numpy releases the interpreter lock in its
    array loops), matmuls on the BLAS threads.  Times are medians of `reps` after one warm-up."""

    def __init__(self, reps):
        import concurrent.futures as cf
        self.cores = os.cpu_count() or 1
        self.blas = int(os.environ.get("OMP_NUM_THREADS", self.cores))
        self.threads = max(1, min(self.cores, self.blas))
        self.pool = cf.ThreadPoolExecutor(self.threads)
        self.reps = reps

    def dequant(self, fn, rows, kdim):
        chunks = np.array_split(rows, min(len(rows), 4 * self.threads))
        return np.concatenate(list(self.pool.map(lambda c: fn(c, kdim), chunks)))

    def median(self, f):
        f()
        ts = []
        for _ in range(self.reps):
            a = time.perf_counter()
            f()
            ts.append(time.perf_counter() - a)
        return float(np.median(ts))

    def gemv(self, fn, rows, kdim, x, total_rows=None, m_scale=1.0):
        """(dequant s, matmul s) for `rows` (a row slice scaled to total_rows when given) times
        x [M, kdim] (an M slice scaled by m_scale)."""
        box = {}
        t_deq = self.median(lambda: box.__setitem__("W", self.dequant(fn, rows, kdim)))
        W = box["W"]
        t_mm = self.median(lambda: x @ W.T)
        r = 1.0 if total_rows is None else total_rows / rows.shape[0]
        return t_deq * r, t_mm * r * m_scale

    def describe(self):
        return {"cores": self.cores, "dequant_threads": self.threads, "blas_threads": self.blas,
                "cpu_model": _cpu_model(), "reps": self.reps}


def cpu_legs(reps, heads_m):
    """CPU baselines of every configuration (BASELINE's plan): configs 1 and 2 and config 5 at
    M=11 in full; config 3 one tensor per (format, shape) on a row slice, summed over the 64-layer
    manifest; configs 4 and 5 at M=2048 (and config 4 at M=8192) on a 256-row M slice and weight-
    row slices, extrapolated linearly."""
    from oracle import quants
    from thunderllamax_amd import formats, synth
    cpu = _Cpu(reps)
    iq3 = quants.dequant_iq3xxs_packed
    q6 = quants.dequant_q6k
    iq4 = quants.dequant_iq4xs
    out = {"host": cpu.describe()}

    # config 1: Q6_K 5120x5120, fp32 x, M=1, in full
    rng = synth.config_rng(1)
    raw = synth.q6k_raw(rng, 5120, 5120)
    x1 = rng.standard_normal((1, 5120)).astype(np.float32)
    td, tm = cpu.gemv(q6, raw, 5120, x1)
    nb1 = 5120 * 210 * 20 + 2 * 4 * 5120
    out["config1"] = {"dequant_s": round(td, 4), "matmul_s": round(tm, 5),
                      "gbs": round(nb1 / (td + tm) / 1e9, 4), "sample": "full matrix"}

    # config 2: IQ3_XXS gate + up 17408x5120 at the headline M, in full
    rng = synth.config_rng(2)
    K, N = 5120, 17408
    pg = formats.iq3_pack_rows(synth.iq3xxs_raw(rng, N, K), K)
    pu = formats.iq3_pack_rows(synth.iq3xxs_raw(rng, N, K), K)
    M = heads_m
    x2 = synth.activations_f16(rng, M, K).astype(np.float32)
    tdg, tmg = cpu.gemv(iq3, pg, K, x2)
    tdu, tmu = cpu.gemv(iq3, pu, K, x2)
    nb2 = 2 * N * 98 * (K // 256) + M * K * 2 + M * N * 2
    t2 = tdg + tdu + tmg + tmu
    out["config2"] = {"M": M, "dequant_s": round(tdg + tdu, 4), "matmul_s": round(tmg + tmu, 4),
                      "gbs": round(nb2 / t2 / 1e9, 4), "sample": "full gate and up matrices"}
    del pg, pu

    # config 3: every (format, shape) of the decode step on a 1024-row slice, x [11, K]
    rng = synth.config_rng(3)
    M3, S = 11, 1024
    manifest = [("iq3", 10240, 5120, 48), ("iq3", 6144, 5120, 48), ("iq3", 48, 5120, 96),
                ("iq3", 5120, 6144, 64), ("iq3", 17408, 5120, 128), ("iq3", 5120, 17408, 64),
                ("iq3", 12288, 5120, 8), ("iq3", 1024, 5120, 32), ("q6", 12288, 5120, 8),
                ("q6", 151936, 5120, 1)]
    t3, w3, per = 0.0, 0, []
    for fmt, n, k, count in manifest:
        rows = min(n, S)
        if fmt == "iq3":
            w = formats.iq3_pack_rows(synth.iq3xxs_raw(rng, rows, k), k)
            td, tm = cpu.gemv(iq3, w, k, synth.activations_f16(rng, M3, k).astype(np.float32), total_rows=n)
            wb = n * 98 * (k // 256)
        else:
            w = synth.q6k_raw(rng, rows, k)
            td, tm = cpu.gemv(q6, w, k, synth.activations_f16(rng, M3, k).astype(np.float32), total_rows=n)
            wb = n * 210 * (k // 256)
        t3 += count * (td + tm)
        w3 += count * wb
        per.append({"tensor": f"{fmt} {n}x{k}", "count": count, "s_each": round(td + tm, 5)})
    out["config3"] = {"M": M3, "s": round(t3, 3), "weight_gbs": round(w3 / t3 / 1e9, 4),
                      "weight_bytes": w3, "per_tensor": per,
                      "sample": f"each tensor on min(rows, {S}) rows, scaled to all rows "
                                "(extrapolated), summed over the 64-layer manifest"}

    # config 4: gate/up and down on 1024-row weight slices, 256-row M slice, extrapolated
    rng = synth.config_rng(4)
    H, F = 5120, 17408
    pg = formats.iq3_pack_rows(synth.iq3xxs_raw(rng, S, H), H)
    pd = formats.iq3_pack_rows(synth.iq3xxs_raw(rng, S, F), F)
    xa = synth.activations_f16(rng, 256, H).astype(np.float32)
    xb = synth.activations_f16(rng, 256, F).astype(np.float32)
    out["config4"] = {}
    for M4 in (2048, 8192):
        tdg, tmg = cpu.gemv(iq3, pg, H, xa, total_rows=2 * F, m_scale=M4 / 256)
        tdd, tmd = cpu.gemv(iq3, pd, F, xb, total_rows=H, m_scale=M4 / 256)
        t4 = tdg + tmg + tdd + tmd
        flops = 2.0 * M4 * H * 2 * F + 2.0 * M4 * F * H
        out["config4"][f"M{M4}"] = {"s": round(t4, 3), "dequant_s": round(tdg + tdd, 3),
                                    "matmul_s": round(tmg + tmd, 3), "tflops": round(flops / t4 / 1e12, 5),
                                    "sample": f"{S}-row weight slices and a 256-row M slice, extrapolated"}

    # config 5: MoE; dequant of 8 experts' slabs scaled to the experts hit, per-pair matmuls
    rng = synth.config_rng(5)
    E, HID, FF = 256, 2048, 512
    sl_gu = np.concatenate([synth.iq4xs_raw(rng, 2 * FF, HID) for _ in range(8)])
    sl_dn = np.concatenate([synth.iq4xs_raw(rng, HID, FF) for _ in range(8)])
    box = {}
    t_deq8 = cpu.median(lambda: box.update(gu=cpu.dequant(iq4, sl_gu, HID), dn=cpu.dequant(iq4, sl_dn, FF)))
    Wgu, Wdn = box["gu"].reshape(8, 2 * FF, HID), box["dn"].reshape(8, HID, FF)
    out["config5"] = {}
    for P in (11, 2048):
        Ps = min(P, 256)
        logits = rng.standard_normal((Ps, E)).astype(np.float32)
        xs = rng.standard_normal((Ps, HID)).astype(np.float32)

        def layer():
            top = np.argsort(-logits, axis=1, kind="stable")[:, :8]
            lg = np.take_along_axis(logits, top, 1)
            g = np.exp(lg - lg[:, :1])
            g /= g.sum(1, keepdims=True)
            y = np.zeros((Ps, HID), dtype=np.float32)
            for e in np.unique(top):
                pos, rank = np.nonzero(top == e)
                w = e % 8      # the 8 dequantized slabs stand for every expert (timing only)
                a = xs[pos] @ Wgu[w].T
                act = a[:, :FF] / (1 + np.exp(-a[:, :FF])) * a[:, FF:]
                y[pos] += g[pos, rank][:, None] * (act @ Wdn[w].T)
            a = xs @ Wgu[0].T                      # the shared expert
            y += (a[:, :FF] / (1 + np.exp(-a[:, :FF])) * a[:, FF:]) @ Wdn[0].T
            return len(np.unique(top))

        with np.errstate(over="ignore"):   # silu of large gate values: exp overflow -> 0, as intended
            hit = layer()
            t_mm = cpu.median(layer) * (P / Ps)
        hit_full = hit if P == Ps else E
        t_deq = t_deq8 * (hit_full + 1) / 8
        t5 = t_deq + t_mm
        flops = 2.0 * 3 * FF * HID * 9 * P
        out["config5"][f"M{P}"] = {"s": round(t5, 4), "dequant_s": round(t_deq, 4), "matmul_s": round(t_mm, 4),
                                   "experts_hit": hit_full, "tflops": round(flops / t5 / 1e12, 5),
                                   "weight_gbs": round((hit_full + 1) * 1671168 / t5 / 1e9, 4),
                                   "sample": ("dequant timed on 8 experts' slabs, scaled to the experts hit + "
                                              "shared; router, per-expert matmuls and combine timed" +
                                              (" on a 256-token slice, extrapolated" if P != Ps else " in full"))}
    return out, cpu


def cpu_baseline_of(legs, cpu):
    """The contract's cpu_baseline object: config 2 (the headline workload), in GB/s."""
    c2 = legs["config2"]
    return {"value": c2["gbs"], "unit": "GB/s", "cores": max(cpu.threads, cpu.blas), "kind": "port",
            "sample": (f"config 2 in full (both {17408}x5120 matrices, M={c2['M']}): numpy dequant on "
                       f"{cpu.threads} threads {c2['dequant_s']:.3f} s + fp32 matmul on {cpu.blas} BLAS threads "
                       f"{c2['matmul_s']:.4f} s, median of {cpu.reps} after one warm-up; host "
                       f"{cpu.describe()['cpu_model']}, {cpu.cores} cores")}


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the hot path is single-GPU; "
              "multi-GPU sharding is a design note). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch
    from thunderllamax_amd import formats, ops, synth

    dev = torch.device("cuda:0")
    if args.sweep_only:
        print(json.dumps({"sweep": sweep_leg(ops, formats, torch, dev, args.steps, args.warmup,
                                             tiled=args.layout == "tiled", per_kind_graphs=False)}), flush=True)
        return
    N, K = 17408, 5120
    ms = [int(m) for m in args.ms.split(",")]
    rng = synth.config_rng(2)
    wbytes = 2 * N * 98 * (K // 256)
    ncopy = max(2, -(-ROT_BYTES // wbytes))
    wsets = []
    for _ in range(ncopy):
        pg = formats.iq3_pack_rows(synth.iq3xxs_raw(rng, N, K), K)
        pu = formats.iq3_pack_rows(synth.iq3xxs_raw(rng, N, K), K)
        wsets.append((torch.from_numpy(pg).to(dev), torch.from_numpy(pu).to(dev)))
    gridf = formats.gridf_tensor(dev)
    # the same weights as tile-major records (repacked on the GPU; same bytes per weight)
    tsets = []
    tbytes = (N + 15) // 16 * 16 * 102 * (K // 256)
    for wg, wu in wsets:
        tg = torch.empty(tbytes, dtype=torch.uint8, device=dev)
        tu = torch.empty(tbytes, dtype=torch.uint8, device=dev)
        ops.pack_iq3_tiled(wg, tg, N, K)
        ops.pack_iq3_tiled(wu, tu, N, K)
        tsets.append((tg, tu))
    # and as packed7 units (the prefill GEMM's plane, which the decode GEMVs also read)
    psets = []
    for wg, wu in wsets:
        pg7 = torch.empty(N * K // 2, dtype=torch.uint8, device=dev)
        pu7 = torch.empty(N * K // 2, dtype=torch.uint8, device=dev)
        ops.pack_w7(wg, pg7, N, K)
        ops.pack_w7(wu, pu7, N, K)
        psets.append((pg7, pu7))
    torch.cuda.synchronize()
    from thunderllamax_amd._lib import LAYOUT_PACK7, LAYOUT_PACKED, LAYOUT_TILED
    layouts = {"tiled": (tsets, LAYOUT_TILED), "packed": (wsets, LAYOUT_PACKED), "pack7": (psets, LAYOUT_PACK7)}
    other = "packed" if args.layout == "tiled" else "tiled"

    def per_m_of(name):
        sets, lay = layouts[name]
        res = {}
        for M in ms:
            x = torch.from_numpy(synth.activations_f16(np.random.default_rng(M), M, K)).to(dev)
            gact = torch.empty(M, N, dtype=torch.float16, device=dev)
            ms_step = time_ffn(ops, sets, gridf, x, gact, args.steps, args.warmup, torch, lay)
            nbytes = wbytes + M * K * 2 + M * N * 2
            gbs = nbytes / (ms_step * 1e-3) / 1e9
            res[str(M)] = {"ms_per_step": round(ms_step, 5), "gbs": round(gbs, 1),
                           "frac_of_peak": round(gbs / PEAK_HBM_GBS, 4),
                           "tflops": round(2 * M * 2 * N * K / (ms_step * 1e-3) / 1e12, 3)}
        return res

    def note(msg):   # progress on stderr: the JSON line stays the only stdout line
        print(f"[bench] {msg}", file=sys.stderr, flush=True)

    small_steps, small_warm = args.steps, args.warmup   # every leg: >= MIN_CALLS calls, >= MIN_WARM warm-ups
    if not args.no_stream:
        note("stream (HBM read ceiling)")
        stream = stream_leg(ops, torch, dev, small_steps, small_warm)
    note(f"ffn8 per M ({args.layout})")
    per_m = per_m_of(args.layout)
    note(f"ffn8 per M ({other})")
    per_m_other = per_m_of(other)
    note("ffn8 per M (pack7)")
    per_m_p7 = per_m_of("pack7")
    head = str(max(ms))
    value = per_m[head]["gbs"]
    for res in (per_m, per_m_other, per_m_p7):
        for r in res.values():
            if MEASURED["hbm_gbs"]:
                r["frac_of_measured"] = round(r["gbs"] / MEASURED["hbm_gbs"], 4)
    out = {
        "metric": "Quant GEMV HBM GB/s (% of peak) at M=1/11; dequant-GEMM TFLOPS at M=2048",
        "value": value,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": per_m[head]["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "iq3_xxs weights, f16 activations, f32 accumulate",
        "data": "synthetic (seeded GGUF IQ3_XXS blocks, bf16->fp16 N(0,1) activations)",
        "config": {"workload": f"IQ3_XXS ffn8 gate+up+SwiGLU GEMV, K={K}, N=2x{N}, M={head}",
                   "M": int(head), "K": K, "N": 2 * N, "weight_bytes": wbytes,
                   "layout": args.layout, "rotation_copies": ncopy, "parallelism": "single GPU"},
        "per_m": per_m,
        "per_m_other_layout": {"layout": other, **per_m_other, "traffic_m11": TRAFFIC.get(f"ffn8_m11_{other}")},
        "per_m_pack7": {"layout": "packed7 units (the prefill GEMM's plane; GGUF bytes counted, the plane "
                                  "holds 128 B per 256 weights)", **per_m_p7,
                        "traffic_m11": TRAFFIC["ffn8_m11_pack7"]},
        "timing": TIMING,
        "roofline": hbm_roofline(
            value,
            ("iq3s_kernel<2,1,8,3> (tiled records, activations staged in LDS)" if args.layout == "tiled" else
             "iq3_gemv_kernel<2,1,4> (+ iq3_xt_kernel for M >= 6)"),
            traffic=TRAFFIC.get(f"ffn8_m{head}_{args.layout}"),
            algorithmic_bytes=wbytes + int(head) * K * 2 + int(head) * N * 2),
    }
    if not args.no_stream:
        out["stream"] = stream
    if not args.no_config1:
        note("config 1 (Q6_K fp32 GEMV)")
        out["config1"] = config1_leg(ops, synth, torch, dev, args.steps, args.warmup)
    gemm_ms = [int(m) for m in str(args.gemm_m).split(",") if int(m) > 0]
    if gemm_ms:
        weights = gemm_weights(formats, synth, torch, dev)
        out["gemm"] = {}
        for i, M in enumerate(gemm_ms):
            note(f"gemm M={M}")
            leg = gemm_leg(ops, formats, synth, torch, dev, M, small_steps, small_warm, weights, w4a8=i == 0)
            if i == 0:   # the metric's M=2048 figures at the top of the object
                out["gemm"].update(leg)
            out["gemm"][f"M{M}"] = {k: v for k, v in leg.items() if k != "w4a8_ffn"}
        del weights
        note(f"merged gemm M={gemm_ms[0]}")
        out["gemm"]["merged"] = merged_gemm_leg(ops, formats, synth, torch, dev, gemm_ms[0], small_steps, small_warm)
    if not args.no_sweep:
        note("sweep (config 3)")
        out["sweep"] = sweep_leg(ops, formats, torch, dev, small_steps, small_warm, tiled=args.layout == "tiled")
    if not args.no_formats:
        note("producers / formats")
        out["producers"] = producers_leg(ops, formats, synth, torch, dev, small_steps, small_warm,
                                         tiled=args.layout == "tiled")
        out["formats"] = formats_leg(ops, synth, torch, dev, small_steps, small_warm)
    if not args.no_moe:
        note("moe (config 5)")
        out["moe"] = moe_leg(ops, formats, synth, torch, dev, small_steps, small_warm)
        note("MoE layer, checkpoint classes")
        out["moe"]["ckpt"] = moe_ckpt_leg(ops, formats, synth, torch, dev, small_steps, small_warm)
    if not args.no_cpu:
        note("CPU baselines")
        legs, cpu = cpu_legs(args.cpu_reps, int(head))
        out["cpu_baseline"] = cpu_baseline_of(legs, cpu)
        out["cpu"] = legs
    if args.copy_mib > 0:
        src = torch.ones(args.copy_mib * 2**18, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
