"""Benchmark of the quantized GEMV/GEMM hot path on one MI355X.

One "step" = one pass of the hot path over one batch-1 input through the
configuration's GEMV set, dispatched as the reference engine runs it: for c1
(the headline, Llama-7B layer shapes, Q4_0) the matrices that share an input
are loaded as one matrix (wqkv = [wq; wk; wv], wgu = [wgate; wup], as
src/model.c:696, 955 concat_mats), so a step is x -> qkv, o, gate_up, down,
lm_head: 5 GEMVs, each on an f32 vector quantized to Q8 first (inside the
GEMV's own launch: the short rows in every workgroup, down (nb = 344) once
per CU in the workgroup-per-CU form; 5 launches, as launches_per_step
reports). The same set as 8 separate GEMVs with 5 separate quantizations
is timed too (ms_per_step_unmerged). Weight copies are rotated so that the
weights streamed per step come from HBM (the copies total >= 2 GB, far above
the 256 MB Infinity Cache). value = weight bytes of the step (the reference's
rows * nb * 18, src/hip.c:1831) / step time, inputs resident in HBM.

The step is captured once per weight copy as a HIP graph and the graphs are
replayed back to back (no host launch per kernel), timed by HIP events on
their stream. roofline describes the step's own launches: each launch of the
step (the same call, the same kernel) timed alone by HIP events on the
stream it runs on, in a graph of that launch repeated over the weight
copies; "achieved" is the algorithmic bytes over the summed durations of the
step's dominant kernel (the one with the largest share of the step's time,
named by the library, amdc_last_kernel), and
"traffic" the HBM bytes per launch of that kernel read live from rocprofv3
FETCH_SIZE / WRITE_SIZE counter passes over the same launches (a child
process under rocprofv3, one pass per counter), scaled by what the counters
read for a copy kernel of known size. Also measured, in "detail": c0 (one
4096x4096 Q4_0 GEMV), c2 (Q4_K 27B shapes), c3 (T = 8 verify GEMV, weights
counted once) and c4 (the T = 256 prefill GEMM on the f16 MFMA and on the
int8 MFMA, TOPS = 2 T rows cols / time), from HIP events around graphs of
back-to-back launches over rotating weight copies.

CPU baseline: the reference's own cpu_gemv_q4 (oracle/_ref/libref_cpu.so,
compiled from hanw/amd.c src/cpu.c), one core, on a bounded sample of the
same c1 step (else the C restatement in oracle/, kind "port").

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1] [--quick] [--no-traffic]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "amd.c_amd"), os.path.join(ROOT, "oracle")]

import amdc  # noqa: E402
from amdc import synth  # noqa: E402

METRIC = "Q4 GEMV weight-read GB/s (% of 8 TB/s HBM) at batch 1; prefill GEMM TOPS"
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
ROTATE_BYTES = 2 << 30


def wbytes(rows, cols, kind=synth.KIND_Q4_0):
    """GGUF weight bytes of a rows x cols matrix (the algorithmic bytes of one GEMV)."""
    return synth.gguf_bytes(kind, rows, cols)


def q8_stride(nb):
    return (40 * nb + 255) // 256 * 256


class Mats:
    """copies x [matrices] of repacked weights on the device."""

    def __init__(self, kind, shapes, seed, min_bytes=ROTATE_BYTES):
        self.kind, self.shapes = kind, shapes
        self.set_bytes = sum(wbytes(r, c, kind) for _, r, c in shapes)
        self.copies = max(1, -(-min_bytes // self.set_bytes))
        host = [amdc.repack(kind, synth.gguf(kind, r, c, seed + i), r, c) for i, (_, r, c) in enumerate(shapes)]
        self.host = host
        self.dev = []
        for _ in range(self.copies):
            self.dev.append([amdc.DevBuf.of(h) for h in host])


def events(n):
    return [amdc.Event() for _ in range(n)]


class Timer:
    """HIP events on one stream around graph replays (the GPU runs a replay without host launches)."""

    def __init__(self):
        self.S = amdc.Stream()
        self.kept = []

    def graph(self, fn):
        # every graph stays alive until the process ends: a profiler's graph-launch hook (rocprofv3
        # --kernel-trace) may still hold a replayed graph when its Python object would be collected,
        # and destroying the executable graph under it is the one use-after-free a run of this file
        # can cause (the library destroys nothing a replay still uses: replay_ms synchronizes first)
        g = amdc.Graph(self.S, fn)
        self.kept.append(g)
        return g

    def replay_ms(self, graphs, reps, warmup=2):
        """ms per replay of the graphs, launched round robin back to back (reps replays)."""
        for i in range(warmup):
            graphs[i % len(graphs)].launch()
        self.S.sync()
        e0, e1 = amdc.Event(), amdc.Event()
        e0.record(self.S.s)
        for i in range(reps):
            graphs[i % len(graphs)].launch()
        e1.record(self.S.s)
        self.S.sync()
        return e0.elapsed_ms(e1) / reps

    def step_ms(self, step, copies, set_bytes, steps, warmup):
        """ms per step: graphs of m consecutive steps (weight copies ci .. ci + m - 1, m chosen so that a
        graph holds about 150 us of GPU work and the host's graph launches stay ahead of the GPU), replayed
        round robin; at least `steps` steps timed (a multiple of m). Returns (ms per step, steps timed)."""
        m = max(1, min(copies, -(-600_000_000 // max(set_bytes, 1))))
        ng = max(1, copies // m)
        graphs = [self.graph(lambda s, k=k: [step((k * m + i) % copies, s) for i in range(m)]) for k in range(ng)]
        reps = -(-steps // m)
        ms = self.replay_ms(graphs, reps, max(1, -(-warmup // m)))
        del graphs
        return ms / m, reps * m

    def per_launch_ms(self, launch, n, reps=4, warmup=2):
        """average ms of one launch: n launches (launch(i, stream)) in one graph, replayed."""
        g = self.graph(lambda s: [launch(i, s) for i in range(n)])
        return self.replay_ms([g], reps, warmup) / n


# ---------------------------------------------------------------- c1 (headline) and c0 / c2 sets

# matrices that read the previous one's input; the reference engine loads each run of them as one
# matrix (wqkv = [wq; wk; wv], wgu = [wgate; wup]: src/model.c:696, 955 concat_mats)
SHARE = {"k", "v", "up", "ffn_up"}


def merged_groups(shapes):
    """[(name, rows, cols, [shape indices])]: runs of shapes with one input, concatenated by rows."""
    out = []
    for i, (name, r, c) in enumerate(shapes):
        if name in SHARE and out:
            n0, r0, c0, idx = out[-1]
            out[-1] = (n0 + "+" + name, r0 + r, c0, idx + [i])
        else:
            out.append((name, r, c, [i]))
    return out


def gemv_set(cfg_name, steps, warmup, seed, timer):
    """A batch-1 GEMV set (c0, c1, c2). The step, as HIP graphs (one per weight copy) replayed:
    - dispatched as the reference engine runs it: the matrices of one input concatenated (wqkv, wgu),
      each GEMV on the f32 vector through amdc_gemv_q4_x / _q4k_x (the quantization fused into the
      GEMV for nb <= 128, else a separate launch) -- ms_per_step;
    - one GEMV per matrix, each input quantized by its own launch -- ms_per_step_unmerged.
    Each GEMV kernel alone: a graph of that GEMV launched back to back over the weight copies."""
    cfg = synth.CONFIGS[cfg_name]
    kind, shapes = cfg["kind"], cfg["shapes"]
    M = Mats(kind, shapes, seed)
    groups = merged_groups(shapes)
    cols_max = max(c for _, _, c in shapes)
    rows_max = max(r for _, r, _, _ in groups)
    X = amdc.DevBuf.of(synth.activations(1, cols_max, seed + 99)[0])
    Q = amdc.DevBuf(q8_stride(cols_max // 32))
    Y = amdc.DevBuf(4 * rows_max)

    def step_unmerged(ci, s):
        for i, (name, r, c) in enumerate(shapes):
            if name not in SHARE:
                amdc.quant_q8(X, Q, c // 32, stream=s)
            amdc.gemv(kind, M.dev[ci][i], Q, Y, r, c // 32, stream=s)

    ms_unmerged, _ = timer.step_ms(step_unmerged, M.copies, M.set_bytes, steps, warmup)
    per, tot = {}, 0.0
    for i, (name, r, c) in enumerate(shapes):
        amdc.quant_q8(X, Q, c // 32)
        t = timer.per_launch_ms(lambda j, s, i=i, r=r, c=c: amdc.gemv(kind, M.dev[j % M.copies][i], Q, Y, r, c // 32, stream=s),
                                M.copies, reps=max(2, steps // 4))
        b = wbytes(r, c)
        per[name] = {"rows": r, "cols": c, "us": round(t * 1e3, 3), "GB/s": round(b / t / 1e6, 1),
                     "hbm_frac": round(b / t / 1e6 / HBM_PEAK_GBS, 4)}
        tot += t
    host = M.host
    del M
    # the merged matrices (row concatenation of the repacked matrices: the layout is row-major)
    G = Mats.__new__(Mats)
    G.set_bytes = sum(wbytes(r, c) for _, r, c, _ in groups)
    G.copies = max(1, -(-ROTATE_BYTES // G.set_bytes))
    hg = [np.concatenate([host[i] for i in idx]) for _, _, _, idx in groups]
    G.dev = [[amdc.DevBuf.of(h) for h in hg] for _ in range(G.copies)]
    del host, hg
    for gi, (name, r, c, _) in enumerate(groups):  # first use sizes the library's workspace, before any capture
        amdc.gemv_x(kind, G.dev[0][gi], X, Y, r, c // 32)

    def step(ci, s):
        for gi, (name, r, c, _) in enumerate(groups):
            amdc.gemv_x(kind, G.dev[ci][gi], X, Y, r, c // 32, stream=s)

    ms_launches, steps_timed = timer.step_ms(step, G.copies, G.set_bytes, steps, warmup)
    # the same step as one GEMV chain launch per weight copy, a grid barrier after each operation
    # (the next one waits for it, as the launches wait for each other); each GEMV quantizes its f32
    # input inside the chain (AMDC_CHAIN_GEMV_X). Both chain kernels: the streaming form (one
    # workgroup per CU, the next operations' weights in flight across the barriers) and the
    # persistent form (2 workgroups per CU).
    ms_chain = {}
    for form, fm in (("streaming", amdc.CHAIN_STREAMING), ("persistent", amdc.CHAIN_PERSISTENT)):
        chains = [amdc.Chain([amdc.chain_gemv_x(kind, G.dev[ci][gi], X, Y, r, c // 32) for gi, (name, r, c, _) in enumerate(groups)],
                             form=fm) for ci in range(G.copies)]
        chains[0].launch()
        chains[0].check()
        ms_chain[form], _ = timer.step_ms(lambda ci, s: chains[ci].launch(s), G.copies, G.set_bytes, steps, warmup)
        chains[0].check()
        del chains
    ms = min(ms_launches, ms_chain["streaming"])
    # each launch of the step alone, the same call as in the step: amdc_gemv_q4_x / _q4k_x (the library
    # quantizes inside the GEMV where it can, else amdc_quant_q8 + the GEMV: two launches in one record)
    launches = []
    for gi, (name, r, c, _) in enumerate(groups):
        nb, b = c // 32, wbytes(r, c, kind)
        amdc.gemv_x(kind, G.dev[0][gi], X, Y, r, nb)
        kname = amdc.last_kernel()  # the kernel the library picked for this shape
        if "_x" not in kname:  # the fused forms are amdc_gemv_*_x1 / _xs<n> / _xw<n>
            kname = "amdc_quant_q8 + " + kname
        t = timer.per_launch_ms(lambda j, s, gi=gi, r=r, nb=nb: amdc.gemv_x(kind, G.dev[j % G.copies][gi], X, Y, r, nb, stream=s),
                                G.copies, reps=max(2, steps // 4))
        launches.append(launch_rec(name, kname, r, c, b, t))
    set_bytes = G.set_bytes
    del G
    kt = {}
    for l in launches:
        kt.setdefault(l["kernel"], [0.0, 0, 0])
        kt[l["kernel"]][0] += l["us"]
        kt[l["kernel"]][1] += l["bytes"]
        kt[l["kernel"]][2] += 1
    dom = max(kt, key=lambda k: kt[k][0])
    launch_us = sum(l["us"] for l in launches)
    return {"set_bytes": set_bytes, "ms_per_step": ms, "steps_timed": steps_timed, "ms_per_step_unmerged": ms_unmerged,
            "ms_per_step_launches": ms_launches, "ms_per_step_chain": ms_chain["streaming"],
            "ms_per_step_chain_persistent": ms_chain["persistent"],
            "step_form": "chain" if ms_chain["streaming"] <= ms_launches else "launches",
            "launches_per_step": sum(2 if l["kernel"].startswith("amdc_quant_q8 + ") else 1 for l in launches),
            "per_shape": per, "step_launches": launches,
            "dominant_kernel": dom, "dominant_launches": kt[dom][2],
            "dominant_bytes_per_launch": kt[dom][1] / kt[dom][2], "dominant_us_per_launch": kt[dom][0] / kt[dom][2],
            "dominant_GBps": kt[dom][1] / kt[dom][0] / 1e3,
            "launches_us_total": launch_us, "launches_GBps": set_bytes / launch_us / 1e3,
            "kernel_GBps_unmerged": set_bytes / tot / 1e6, "weight_copies": -(-ROTATE_BYTES // set_bytes)}


def launch_rec(op, kernel, rows, cols, b, t_ms):
    us = t_ms * 1e3
    return {"op": op, "kernel": kernel, "rows": rows, "cols": cols, "weight_bytes": b, "bytes": b, "us": round(us, 3),
            "GB/s": round(b / us / 1e3, 1) if b else None, "hbm_frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4) if b else None}


def verify_set(steps, seed, timer):
    """c3: T = 8 vectors against each matrix (weights read once per launch); also T = 16 (the
    16-vector kernels, one launch)."""
    cfg = synth.CONFIGS["c3"]
    T = cfg["T"]
    out = {}
    for i, (name, r, c, kind) in enumerate(cfg["shapes"]):
        M = Mats(kind, [(name, r, c)], seed + i, min_bytes=1 << 30)
        nb = c // 32
        xs = q8_stride(nb)
        X = amdc.DevBuf.of(synth.activations(16, c, seed + 50 + i))
        Q = amdc.DevBuf(16 * xs)
        Y = amdc.DevBuf(4 * 16 * r)
        amdc.quant_q8(X, Q, nb, 16, 4 * c, xs)
        ts = {}
        for tn in (T, 16):
            amdc.gemv_t(kind, M.dev[0][0], Q, Y, r, nb, tn, xs, r)  # sizes the library's workspace before the capture
            ts[tn] = timer.per_launch_ms(lambda j, s: amdc.gemv_t(kind, M.dev[j % M.copies][0], Q, Y, r, nb, tn, xs, r, stream=s),
                                         M.copies)
        t = ts[T]
        b = wbytes(r, c)
        out[name] = {"rows": r, "cols": c, "T": T, "us": round(t * 1e3, 3), "GB/s": round(b / t / 1e6, 1),
                     "hbm_frac": round(b / t / 1e6 / HBM_PEAK_GBS, 4), "T16_us": round(ts[16] * 1e3, 3)}
        del M
    return out


def prefill_set(steps, seed, timer):
    """c4: the T = 256 prefill GEMM, TOPS = 2 T rows cols / time."""
    cfg = synth.CONFIGS["c4"]
    T = cfg["T"]
    out = {}
    for i, (name, r, c) in enumerate(cfg["shapes"]):
        M = Mats(cfg["kind"], [(name, r, c)], seed + i, min_bytes=1 << 30)
        nb = c // 32
        xs = q8_stride(nb)
        X = amdc.DevBuf.of(synth.activations(T, c, seed + 70 + i))
        Q = amdc.DevBuf(T * xs)
        Y = amdc.DevBuf(4 * T * r)
        amdc.quant_q8(X, Q, nb, T, 4 * c, xs)
        amdc.gemm_q4k(M.dev[0][0], Q, Y, r, nb, T, xs, r)  # sizes the library's workspace before the capture
        # 4 untimed replays first (about 13 ms of GEMMs): the first GEMMs a process runs measured about 3 %
        # slower than the same graph replayed later
        t = timer.per_launch_ms(lambda j, s: amdc.gemm_q4k(M.dev[j % M.copies][0], Q, Y, r, nb, T, xs, r, stream=s), M.copies, reps=4,
                                warmup=4)
        tops = 2.0 * T * r * c / t / 1e9
        out[name] = {"rows": r, "cols": c, "T": T, "us": round(t * 1e3, 3), "TOPS": round(tops, 1),
                     "int8_mfma_frac": round(tops / INT8_PEAK_TOPS, 4), "kernel": "f16 MFMA (default)"}
        # the int8-MFMA kernel (tuning gemm_kernel 2: 64 rows x 128 tokens, 1: x 64 tokens) beside it
        for kk, label in ((2, "int8_n128"), (1, "int8_n64")):
            amdc.set_tuning(gemm_kernel=kk)
            t8 = timer.per_launch_ms(lambda j, s: amdc.gemm_q4k(M.dev[j % M.copies][0], Q, Y, r, nb, T, xs, r, stream=s), M.copies, reps=2)
            amdc.set_tuning()
            out[name][label] = {"us": round(t8 * 1e3, 3), "TOPS": round(2.0 * T * r * c / t8 / 1e9, 1),
                                "int8_mfma_frac": round(2.0 * T * r * c / t8 / 1e9 / INT8_PEAK_TOPS, 4)}
        del M
    return out


def ceiling_set(seed, timer):
    """The practical ceiling of each decode launch: a plain read (amdc_probe_read, 16-byte loads, 4 in
    flight per lane, the best of several grid sizes) of exactly the launch's weight bytes, timed like
    the GEMVs (one graph of back-to-back launches over rotating copies of >= 1 GB), beside the GEMV on
    a Q8 vector (amdc_gemv_q4 / _q4k) and on the f32 vector (amdc_gemv_q4_x / _q4k_x, the step's call),
    for the merged matrices of the c0 / c1 / c2 steps."""
    out = {}
    scratch = amdc.DevBuf(4 * 65536)
    for cname in ("c1", "c2"):
        cfg = synth.CONFIGS[cname]
        kind = cfg["kind"]
        for gi, (name, r, c, _) in enumerate(merged_groups(cfg["shapes"])):
            if (r, c) in [(v["rows"], v["cols"]) for v in out.values()]:
                continue
            nb, b = c // 32, wbytes(r, c, kind)
            M = Mats(kind, [(name, r, c)], seed + gi, min_bytes=1 << 30)
            X = amdc.DevBuf.of(synth.activations(1, c, seed + 7)[0])
            Q, Y = amdc.DevBuf(q8_stride(nb)), amdc.DevBuf(4 * r)
            amdc.quant_q8(X, Q, nb)
            rd = {}
            for grid in (256, 512, 1024, 2048, 4096):
                rd[grid] = timer.per_launch_ms(lambda j, s, g=grid: amdc.probe_read(M.dev[j % M.copies][0], b // 16 * 16, scratch, g,
                                                                                    stream=s), M.copies)
            grid = min(rd, key=rd.get)
            tq = timer.per_launch_ms(lambda j, s: amdc.gemv(kind, M.dev[j % M.copies][0], Q, Y, r, nb, stream=s), M.copies)
            kq = amdc.last_kernel()
            amdc.gemv_x(kind, M.dev[0][0], X, Y, r, nb)
            kx = amdc.last_kernel()
            if "_x" not in kx:
                kx = "amdc_quant_q8 + " + kx
            tx = timer.per_launch_ms(lambda j, s: amdc.gemv_x(kind, M.dev[j % M.copies][0], X, Y, r, nb, stream=s), M.copies)
            us = lambda t: round(t * 1e3, 3)
            out[f"{cname}:{name}"] = {"rows": r, "cols": c, "bytes": b, "read_us": us(rd[grid]), "read_grid": grid,
                                      "read_hbm_frac": round(b / rd[grid] / 1e6 / HBM_PEAK_GBS, 4),
                                      "gemv_q8_us": us(tq), "gemv_q8_kernel": kq, "gemv_q8_of_read": round(rd[grid] / tq, 3),
                                      "gemv_f32_us": us(tx), "gemv_f32_kernel": kx, "gemv_f32_of_read": round(rd[grid] / tx, 3)}
            del M
    return out


def k8_set(seed, timer):
    """The Q8_0 and Q6_K decode GEMVs at the sizes they have in the c1 / c2 models (the Q6_K
    matrices of a Q4_K_M file: ffn_down, attn_v, lm_head; Q8_0 projections): us per launch and the
    GGUF weight bytes per second, at T = 1 and for the T = 8 verify (weights read once); TOPS of the
    T = 256 prefill GEMM on the ffn-sized ones."""
    out = {}
    sets = [(synth.KIND_Q8_0, "q8_0_q", 4096, 4096), (synth.KIND_Q8_0, "q8_0_gate", 11008, 4096),
            (synth.KIND_Q8_0, "q8_0_down", 4096, 11008), (synth.KIND_Q6_K, "q6_k_ffn_down", 5120, 17408),
            (synth.KIND_Q6_K, "q6_k_attn_v", 1024, 5120), (synth.KIND_Q6_K, "q6_k_lm_head", 152064, 5120)]
    for i, (kind, name, r, c) in enumerate(sets):
        M = Mats(kind, [(name, r, c)], seed + i, min_bytes=1 << 30)
        nb, xs = c // 32, q8_stride(c // 32)
        X = amdc.DevBuf.of(synth.activations(8, c, seed + 90 + i))
        Q, Y = amdc.DevBuf(8 * xs), amdc.DevBuf(4 * 8 * r)
        amdc.quant_q8(X, Q, nb, 8, 4 * c, xs)
        t = timer.per_launch_ms(lambda j, s: amdc.gemv(kind, M.dev[j % M.copies][0], Q, Y, r, nb, stream=s), M.copies)
        amdc.gemv_t(kind, M.dev[0][0], Q, Y, r, nb, 8, xs, r)  # sizes the workspace before the capture
        t8 = timer.per_launch_ms(lambda j, s: amdc.gemv_t(kind, M.dev[j % M.copies][0], Q, Y, r, nb, 8, xs, r, stream=s), M.copies)
        b = wbytes(r, c, kind)
        out[name] = {"rows": r, "cols": c, "us": round(t * 1e3, 3), "GB/s": round(b / t / 1e6, 1),
                     "hbm_frac": round(b / t / 1e6 / HBM_PEAK_GBS, 4), "T8_us": round(t8 * 1e3, 3),
                     "T8_GB/s": round(b / t8 / 1e6, 1)}
        if r * c >= 4096 * 11008 and r * c < 10 ** 9:  # the prefill GEMM at T = 256 on the ffn-sized matrices
            T = 256
            X2 = amdc.DevBuf.of(synth.activations(T, c, seed + 95 + i))
            Q2, Y2 = amdc.DevBuf(T * xs), amdc.DevBuf(4 * T * r)
            amdc.quant_q8(X2, Q2, nb, T, 4 * c, xs)
            amdc.gemm(kind, M.dev[0][0], Q2, Y2, r, nb, T, xs, r)  # sizes the workspace before the capture
            tg = timer.per_launch_ms(lambda j, s: amdc.gemm(kind, M.dev[j % M.copies][0], Q2, Y2, r, nb, T, xs, r, stream=s), M.copies, reps=2)
            out[name].update({"T256_us": round(tg * 1e3, 1), "T256_TOPS": round(2.0 * T * r * c / tg / 1e9, 1)})
            del X2, Q2, Y2
        del M
    return out


def load_set(seed):
    """The load of quantized matrices from a GGUF file (amdc_gguf_load: host repack in row chunks
    on threads into pinned buffers, async copies to the device) against the host repack alone on
    one thread (the reference's load-time repack_q4k / repack_q6k is single-threaded): GB/s of GGUF
    bytes, the file in the page cache (read once before timing)."""
    import tempfile
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import gguf_writer as gw
    shapes = [("ffn_up", synth.KIND_Q4_K, 17408, 5120), ("ffn_down", synth.KIND_Q6_K, 5120, 17408),
              ("attn_q", synth.KIND_Q8_0, 5120, 5120)]
    tensors, total = [], 0
    for i, (name, kind, r, c) in enumerate(shapes):
        src = synth.gguf(kind, r, c, seed + i)
        tensors.append((name, synth.GGML[kind], (c, r), src.tobytes()))
        total += src.size
    out = {}
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "bench.gguf")
        gw.write(path, [("general.architecture", gw.STR, "bench")], tensors)
        del tensors
        with amdc.Gguf(path) as g:
            for name, _, _, _ in shapes:  # page the file in
                g.repack(name, 0)
            t0 = time.perf_counter()
            for name, _, _, _ in shapes:
                g.repack(name, 1)
            t_one = time.perf_counter() - t0
            mats = []
            amdc.sync()
            t0 = time.perf_counter()
            for name, _, _, _ in shapes:
                mats.append(g.load(name, 0))
            amdc.sync()
            t_load = time.perf_counter() - t0
            for m in mats:
                m.free()
    out = {"gguf_bytes": total, "host_repack_1thread_GBps": round(total / t_one / 1e9, 2),
           "load_to_device_GBps": round(total / t_load / 1e9, 2), "load_ms": round(t_load * 1e3, 1),
           "matrices": [f"{n} {synth.GGML[k]} {r}x{c}" for n, k, r, c in shapes]}
    return out


# ---------------------------------------------------------------- CPU baseline

def producers_set(timer):
    """The fused Q8 producers at the c1/c2 sizes: us per launch (graphs of back-to-back launches)."""
    out = {}
    g = np.random.default_rng(7)
    for name, n in (("rmsnorm_q8", 4096), ("rmsnorm_q8", 5120), ("swiglu_q8", 11008), ("swiglu_q8", 17408)):
        nb = n // 32
        X = amdc.DevBuf.of(g.standard_normal(n).astype(np.float32))
        Wt = amdc.DevBuf.of(np.ones(n, np.float32))
        Y, Q = amdc.DevBuf(4 * n), amdc.DevBuf(q8_stride(nb))
        if name == "rmsnorm_q8":
            t = timer.per_launch_ms(lambda j, s: amdc.rmsnorm_q8(X, Wt, Y, n, 1e-6, Q, stream=s), 64)
        else:
            t = timer.per_launch_ms(lambda j, s: amdc.swiglu_q8(X, Wt, n, Q, stream=s), 64)
        out[f"{name}_{n}"] = {"us": round(t * 1e3, 3)}
    # the decode GEMV with the fused RMSNorm tail (amdc_gemv_norm) against the GEMV and a separate
    # amdc_rmsnorm_q8 launch, over rotating weight copies (HBM), on the c1 o and c2 attn_out shapes
    for kind, r, c in ((synth.KIND_Q4_0, 4096, 4096), (synth.KIND_Q4_K, 5120, 6144)):
        nb = c // 32
        M = Mats(kind, [("w", r, c)], 70 + r, min_bytes=1 << 30)
        X = amdc.DevBuf.of(g.standard_normal(c).astype(np.float32))
        Q, Y = amdc.DevBuf(q8_stride(nb)), amdc.DevBuf(4 * r)
        amdc.quant_q8(X, Q, nb)
        Wn, Ny, Nq = amdc.DevBuf.of(np.ones(r, np.float32)), amdc.DevBuf(4 * r), amdc.DevBuf(q8_stride(r // 32))

        def two(j, s):
            amdc.gemv(kind, M.dev[j % M.copies][0], Q, Y, r, nb, stream=s)
            amdc.rmsnorm_q8(Y, Wn, Ny, r, 1e-6, Nq, stream=s)

        t2 = timer.per_launch_ms(two, M.copies)
        t1 = timer.per_launch_ms(lambda j, s: amdc.gemv_norm(kind, M.dev[j % M.copies][0], Q, Y, r, nb, Wn, Ny, 1e-6, nq=Nq, stream=s),
                                 M.copies)
        out[f"gemv_norm_{r}x{c}"] = {"fused_us": round(t1 * 1e3, 3), "gemv_then_rmsnorm_us": round(t2 * 1e3, 3)}
        del M
    return out


def cpu_baseline(seed, budget_s=12.0):
    """The c1 step on one host core: reference cpu_gemv_q4 (oracle/_ref) or the restatement."""
    from oracle import GGML_Q4_0, Oracle, RefCPU

    shapes = synth.CONFIGS["c1"]["shapes"]
    x = synth.activations(1, 11008, seed + 99)[0]
    srcs = [synth.gguf(synth.KIND_Q4_0, r, c, seed + i) for i, (_, r, c) in enumerate(shapes)]
    if RefCPU.available():
        ref = RefCPU()
        kind = "reference"
        mats = [ref.mat(GGML_Q4_0, s, r, c) for s, (_, r, c) in zip(srcs, shapes)]
        xq = {c: ref.quant_q8(x[:c]) for _, _, c in shapes}

        def run():
            for m, (_, r, c) in zip(mats, shapes):
                m.gemv(xq[c])
    else:
        orc = Oracle()
        kind = "port"
        arrs = [orc.repack(GGML_Q4_0, s, r, c // 32) for s, (_, r, c) in zip(srcs, shapes)]
        xq = {c: orc.quant_q8(x[:c]) for _, _, c in shapes}

        def run():
            for (qw, qs), (_, r, c) in zip(arrs, shapes):
                orc.gemv(GGML_Q4_0, qw, qs, r, c // 32, xq[c])
    set_bytes = sum(wbytes(r, c) for _, r, c in shapes)
    n, t0 = 0, time.perf_counter()
    while True:
        run()
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 50:
            break
    return {"value": round(set_bytes * n / el / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": kind,
            "sample": f"{n} c1 steps (8 Q4_0 GEMVs, {set_bytes / 1e6:.1f} MB of weights each) in {el:.1f} s, single thread, "
                      f"{'cpu_gemv_q4 of hanw/amd.c src/cpu.c' if kind == 'reference' else 'oracle/amdc_oracle.c'}"}


def cpu_baseline_rows(seed, budget_s=6.0):
    """The same c1 step on the host's cores: the restatement's row-parallel GEMV (the same per-row
    arithmetic as cpu_gemv_q4, so the same bits), one thread per core up to 16 (the GPU box's CPU
    share). A second baseline, reported beside the one-core one."""
    from oracle import GGML_Q4_0, Oracle

    cores = min(16, len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1))
    shapes = synth.CONFIGS["c1"]["shapes"]
    x = synth.activations(1, 11008, seed + 99)[0]
    orc = Oracle()
    arrs = [orc.repack(GGML_Q4_0, synth.gguf(synth.KIND_Q4_0, r, c, seed + i), r, c // 32) for i, (_, r, c) in enumerate(shapes)]
    xq = {c: orc.quant_q8(x[:c]) for _, _, c in shapes}
    set_bytes = sum(wbytes(r, c) for _, r, c in shapes)
    n, t0 = 0, time.perf_counter()
    while True:
        for (qw, qs), (_, r, c) in zip(arrs, shapes):
            orc.gemv(GGML_Q4_0, qw, qs, r, c // 32, xq[c], threads=cores)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 200:
            break
    return {"value": round(set_bytes * n / el / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"{n} c1 steps in {el:.1f} s, {cores} threads, oracle/amdc_oracle.c row-parallel (bit-identical to cpu_gemv_q4)"}


# ---------------------------------------------------------------- HBM traffic (rocprofv3 counters, live)

CAL_BYTES = 256 << 20


def traffic_child(seed):
    """Run under rocprofv3 --pmc by measure_traffic: the probe copy of CAL_BYTES twice (the counters'
    yardstick), then each launch of the c1 step 3 times, eager (one copy of the merged matrices)."""
    amdc.open_device()
    A, B = amdc.DevBuf(CAL_BYTES), amdc.DevBuf(CAL_BYTES)
    A.fill(1)
    for _ in range(2):
        amdc.probe_copy(B, A, CAL_BYTES, 4096)
    amdc.sync()
    del A, B
    kind = synth.CONFIGS["c1"]["kind"]
    groups = merged_groups(synth.CONFIGS["c1"]["shapes"])
    W = [amdc.DevBuf.of(amdc.repack(kind, synth.gguf(kind, r, c, seed + i), r, c)) for i, (_, r, c, _) in enumerate(groups)]
    cols_max = max(c for _, _, c, _ in groups)
    X = amdc.DevBuf.of(synth.activations(1, cols_max, seed + 99)[0])
    Q, Y = amdc.DevBuf(q8_stride(cols_max // 32)), amdc.DevBuf(4 * max(r for _, r, _, _ in groups))
    for gi, (_, r, c, _) in enumerate(groups):
        for _ in range(3):
            amdc.gemv_x(kind, W[gi], X, Y, r, c // 32)
    amdc.sync()


def measure_traffic(seed, kernel):
    """HBM bytes per launch of `kernel` in the c1 step: two rocprofv3 --pmc passes (FETCH_SIZE, then
    WRITE_SIZE, KiB per dispatch) over traffic_child, each counter scaled by what it reads for the probe
    copy (CAL_BYTES read, CAL_BYTES written). Returns (bytes per launch, details) or (None, reason)."""
    import csv
    import shutil
    import subprocess
    import tempfile

    if shutil.which("rocprofv3") is None:
        return None, "rocprofv3 not found"
    per = {}
    for ctr in ("FETCH_SIZE", "WRITE_SIZE"):
        d = tempfile.mkdtemp(prefix="amdc_pmc_", dir="/tmp")
        cmd = ["rocprofv3", "--pmc", ctr, "-d", d, "-o", "t", "--output-format", "csv", "--",
               sys.executable, os.path.abspath(__file__), "--traffic-child", "--seed", str(seed)]
        try:
            r = subprocess.run(cmd, cwd="/tmp", env={**os.environ, "TMPDIR": "/tmp"}, capture_output=True, text=True, timeout=240)
        except subprocess.TimeoutExpired:
            return None, f"rocprofv3 --pmc {ctr} timed out"
        files = [os.path.join(dp, f) for dp, _, fs in os.walk(d) for f in fs if f.endswith("counter_collection.csv")]
        if r.returncode != 0 or not files:
            return None, f"rocprofv3 --pmc {ctr} failed (rc {r.returncode}): {(r.stderr or '')[-300:]}"
        vals = {}
        for row in csv.DictReader(open(files[0])):
            if row["Counter_Name"] == ctr:
                vals.setdefault(row["Kernel_Name"], []).append(float(row["Counter_Value"]))
        shutil.rmtree(d, ignore_errors=True)
        cal = vals.get("amdc_probe_copy")
        mine = vals.get(kernel.split(" + ")[-1])  # a quantize + GEMV record: the GEMV's counters
        if not cal or not mine:
            return None, f"{ctr}: no dispatches of amdc_probe_copy / {kernel} in the counter output"
        scale = CAL_BYTES / (sum(cal) / len(cal) * 1024.0)
        per[ctr] = {"KiB_per_dispatch": round(sum(mine) / len(mine), 1), "scale": round(scale, 4),
                    "bytes_per_launch": sum(mine) / len(mine) * 1024.0 * scale, "dispatches": len(mine)}
    total = per["FETCH_SIZE"]["bytes_per_launch"] + per["WRITE_SIZE"]["bytes_per_launch"]
    return total, per


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--seed", type=int, default=2024)
    ap.add_argument("--quick", action="store_true", help="headline only (no c0/c2/c3/c4 detail, no CPU baseline)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--sets", default="c0,c2,c3,c4,producers,ceiling,k8,load",
                    help="detail sets to run after the headline (comma list of c0, c2, c3, c4, producers, ceiling, k8, load)")
    ap.add_argument("--calibrate", action="store_true",
                    help="first run the probe copy kernel over 256 MiB 3 times (the FETCH_SIZE / WRITE_SIZE yardstick)")
    ap.add_argument("--no-traffic", action="store_true", help="no rocprofv3 counter passes (roofline.traffic null)")
    ap.add_argument("--traffic-child", action="store_true", help=argparse.SUPPRESS)
    a = ap.parse_args()
    if a.traffic_child:
        traffic_child(a.seed)
        return
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU; across GPUs the GEMV path would shard each matrix by rows "
              "(no multi-GPU run is built). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    amdc.open_device()
    print(f"bench: {amdc.cu_count()} CUs", file=sys.stderr, flush=True)
    if a.calibrate:
        n = 256 << 20
        A, B = amdc.DevBuf(n), amdc.DevBuf(n)
        A.fill(1)
        for _ in range(3):
            amdc.probe_copy(B, A, n, 4096)
        amdc.sync()
        del A, B

    timer = Timer()
    c1 = gemv_set("c1", a.steps, a.warmup, a.seed, timer)
    value = c1["set_bytes"] / (c1["ms_per_step"] * 1e-3) / 1e9
    print(f"bench: c1 {value:.1f} GB/s per step, {c1['dominant_kernel']} {c1['dominant_GBps']:.1f} GB/s, "
          f"launches alone {c1['launches_GBps']:.1f} GB/s", file=sys.stderr, flush=True)
    detail = {"c1": c1}
    sets = set() if a.quick else set(a.sets.split(","))
    for name in ("c0", "c2"):
        if name in sets:
            detail[name] = gemv_set(name, a.steps, 2, a.seed + 1000, timer)
            print(f"bench: {name} {detail[name]['set_bytes'] / detail[name]['ms_per_step'] / 1e6:.1f} GB/s per step, "
                  f"launches alone {detail[name]['launches_GBps']:.1f} GB/s", file=sys.stderr, flush=True)
    for key, name, fn in (("c3", "c3", lambda: verify_set(a.steps, a.seed + 2000, timer)),
                          ("c4", "c4", lambda: prefill_set(a.steps, a.seed + 3000, timer)),
                          ("producers", "producers", lambda: producers_set(timer)),
                          ("ceiling", "decode_ceiling", lambda: ceiling_set(a.seed + 6000, timer)),
                          ("k8", "q8_0_q6_k", lambda: k8_set(a.seed + 4000, timer)),
                          ("load", "gguf_load", lambda: load_set(a.seed + 5000))):
        if key in sets:
            detail[name] = fn()
            print(f"bench: {name} {json.dumps(detail[name])}", file=sys.stderr, flush=True)
    cpu = None
    if not a.quick and not a.no_cpu:
        cpu = cpu_baseline(a.seed)
        print(f"bench: cpu {json.dumps(cpu)}", file=sys.stderr, flush=True)
        detail["cpu_all_cores"] = cpu_baseline_rows(a.seed)
        print(f"bench: cpu_all_cores {json.dumps(detail['cpu_all_cores'])}", file=sys.stderr, flush=True)
    traffic, tinfo = (None, "not measured (--no-traffic or --quick)") if (a.no_traffic or a.quick) else \
        measure_traffic(a.seed, c1["dominant_kernel"])
    print(f"bench: traffic {traffic} {json.dumps(tinfo)}", file=sys.stderr, flush=True)
    ach = c1["dominant_GBps"]
    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": c1["steps_timed"],
        "warmup": a.warmup,
        "ms_per_step": round(c1["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded: uniform nibbles, f16 |N(0,1)|*0.02 scales, N(0,1) activations)",
        "config": {"workload": "c1: Llama-7B layer GEMV set, Q4_0 x Q8, batch 1 (q,k,v,o 4096x4096; gate,up 11008x4096; "
                               "down 4096x11008; lm_head 32000x4096), f32 inputs quantized to Q8 in the step; q,k,v and "
                               "gate,up run as the concatenated wqkv 12288x4096 and wgu 22016x4096 (src/model.c:696,955)",
                   "launches_per_step": c1["launches_per_step"], "ms_per_step_unmerged": round(c1["ms_per_step_unmerged"], 4),
                   "weight_bytes_per_step": c1["set_bytes"], "rotation_copies_bytes": ROTATE_BYTES, "batch": 1},
        "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": round(traffic) if traffic else None,
                     "kernel": c1["dominant_kernel"], "launches_per_step": c1["dominant_launches"],
                     "algorithmic_bytes_per_launch": round(c1["dominant_bytes_per_launch"]),
                     "us_per_launch": round(c1["dominant_us_per_launch"], 3), "traffic_counters": tinfo},
        "cpu_baseline": cpu,
        "detail": detail,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
