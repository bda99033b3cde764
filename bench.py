#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-matmul hot path (libdeepinfer_hip) on one GPU.

Headline (the JSON `value`): config 2 of BASELINE.json, one decode MoE step for one token
(8-bit g64, 256 experts top-8, hidden 2048, intermediate 512, shared expert with a
sigmoid gate) as achieved HBM GB/s of its algorithmic bytes. The other configs are
measured in the same run and reported under "secondary". Weights and activations are
seeded synthetic data created on the GPU; every timed step reads weights that are not
resident in the 256 MB Infinity Cache (rotating copies whose working set between reuses
exceeds 512 MB). The timed loop (exactly --steps steps) is captured in a HIP graph and
replayed between two synchronizations; `value` and `ms_per_step` come from that wall
clock. Per-kernel durations come from HIP event pairs that the library records on the
launch stream around every kernel (hipExtLaunchKernelGGL start/stop events) while the
same steps run again directly after the timed replay; `roofline.achieved` is the dominant
kernel's algorithmic bytes per launch over its average duration. `roofline.traffic` is
the HBM bytes per launch that rocprofv3 --pmc FETCH_SIZE + WRITE_SIZE measured for that
kernel, scaled by the counters' reading for a plain copy of known size, read from the
summaries committed under profiles/ (null when none is present). `roofline.kernels` gives
every decode kernel's fraction from these events and from the rocprofv3 kernel-trace
average committed under profiles/ (`frac_rocprof`; the dominant kernel's is also
`roofline.frac_rocprof`).

python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload all|decode|qmv|prefill|
                 prefill5|dense|lm_head|peaks|copycal|decode_timeline] [--layers L]
                [--cpu-seconds S] [--no-cpu]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "infer.net_amd"))

PEAK_HBM_GBS = 8000.0        # MI355X HBM3E
PEAK_BF16_TFLOPS = 2500.0    # MI355X dense bf16 MFMA
H, E, I = 2048, 256, 512


def metric_name():
    try:
        with open(os.path.join(ROOT, "BASELINE.json")) as f:
            return json.load(f)["metric"]
    except Exception:
        return "decode qmv HBM GB/s (% peak); prefill MoE qmm TFLOP/s (% MFMA peak); tok/s"


def qbytes(experts, rows, cols, bits):
    """Algorithmic bytes of a packed matrix: codes + bf16 scale + bf16 bias per 64."""
    return experts * rows * (cols * bits // 8 + (cols // 64) * 4)


def traffic_from_profiles(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 --pmc summaries
    (a line `traffic_bytes_per_launch[<kernel>]: <bytes>` in profiles/*.md), else None."""
    import glob
    import re
    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", "*.md"))):
        with open(path) as f:
            for line in f:
                m = re.match(r"\s*traffic_bytes_per_launch\[([^\]]+)\]:\s*([0-9.eE+]+)", line)
                if m and m.group(1) == kernel:
                    return float(m.group(2))
    return None


def rocprof_avg_us_from_profiles(kernel):
    """Average duration (us) of `kernel` from the committed rocprofv3 --kernel-trace summaries
    (a line `rocprof_avg_us[<kernel>]: <us>` in profiles/*.md), else None."""
    import glob
    import re
    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", "*.md"))):
        with open(path) as f:
            for line in f:
                m = re.match(r"\s*rocprof_avg_us\[([^\]]+)\]:\s*([0-9.eE+]+)", line)
                if m and m.group(1) == kernel:
                    return float(m.group(2))
    return None


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class Bench:
    def __init__(self, args):
        import torch
        import deepinfer_hip as dh
        self.torch, self.dh, self.args = torch, dh, args
        torch.cuda.init()
        self.dev = dh.QuantizedHip()
        self.gen = torch.Generator(device="cuda")
        self.gen.manual_seed(0)
        self.keep = []

    # ---------------------------------------------------------------- synthetic data
    def matrix(self, experts, rows, cols, bits, scale=(5e-4, 2e-3)):
        torch, dh = self.torch, self.dh
        m = self.dev.allocate(experts, rows, cols, bits)
        n_bytes = experts * rows * cols * bits // 8
        step = 1 << 28
        for off in range(0, n_bytes, step):
            n = min(step, n_bytes - off)
            codes = torch.randint(0, 256, (n,), dtype=torch.uint8, device="cuda", generator=self.gen)
            m.upload_from(0, codes, off)
            del codes
        ng = experts * rows * (cols // 64)
        s = torch.empty(ng, device="cuda").uniform_(scale[0], scale[1], generator=self.gen).to(torch.bfloat16)
        b = (-(1 << (bits - 1)) * s.float() + 1e-4 * torch.randn(ng, device="cuda", generator=self.gen)).to(torch.bfloat16)
        m.upload_from(1, s)
        m.upload_from(2, b)
        return m

    def bf16(self, *shape):
        return self.torch.randn(*shape, device="cuda", generator=self.gen).to(self.torch.bfloat16)

    def moe_layer(self, bits, with_router=True):
        dh = self.dh
        mats = dict(
            router=self.matrix(1, E, H, 8, scale=(1.25e-4, 5e-4)) if with_router else None,
            gate=self.matrix(E, I, H, bits), up=self.matrix(E, I, H, bits), down=self.matrix(E, H, I, bits),
            shared_gate=self.matrix(1, I, H, bits), shared_up=self.matrix(1, I, H, bits),
            shared_down=self.matrix(1, H, I, bits), shared_route=self.matrix(1, 1, H, 8))
        self.keep.append(mats)
        return mats, dh.make_layer(mats["router"], mats["gate"], mats["up"], mats["down"], mats["shared_gate"],
                                   mats["shared_up"], mats["shared_down"], mats["shared_route"])

    # ---------------------------------------------------------------- timing helper
    def timed_graph(self, step_fn, steps, warmup):
        """Runs `warmup` eager steps, captures exactly `steps` steps into one HIP graph,
        replays it once untimed, then times one replay between two synchronizations
        (wall clock). Then the same `steps` steps run eagerly with the library's per-stage
        HIP events, queued behind a GPU sleep so that the host enqueues ahead and the
        kernels execute back to back as in the graph. Returns (ms per step,
        {stage: (ms total, launches)})."""
        torch, dh = self.torch, self.dh
        # at least one eager step: scratch buffers must exist before capture
        for i in range(max(1, warmup)):
            step_fn(i)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            with torch.cuda.graph(g, stream=stream):
                for i in range(steps):
                    step_fn(i)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        g.replay()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        del g
        # (at most 96 profiled steps so that the queued work fits the hardware queue and
        # nothing waits on the host once the sleep ends)
        nprof = min(steps, 96)
        dh.set_profiling(self.dev, True)
        torch.cuda._sleep(int(2.4e9 * max(0.01, nprof * 60e-6)))
        for i in range(nprof):
            step_fn(i)
        prof = dh.profile_read(self.dev)
        torch.cuda.synchronize()
        dh.set_profiling(self.dev, False)
        return (t1 - t0) * 1e3 / steps, prof

    # ---------------------------------------------------------------- workloads
    def decode(self, steps, warmup, layers=24):
        """Config 2: decode MoE step, 8-bit, rotating `layers` layer copies (each ~855 MB)."""
        torch, dh = self.torch, self.dh
        log(f"[decode] building {layers} MoE layers (8-bit)")
        built = [self.moe_layer(8) for _ in range(layers)]
        xs = self.bf16(64, H)
        res = self.bf16(H)

        def step(i):
            dh.moe_decode(self.dev, built[i % layers][1], xs[i % 64], res)

        ms, prof = self.timed_graph(step, steps, warmup)
        w_bytes = 9 * (2 * qbytes(1, I, H, 8) + qbytes(1, H, I, 8)) + qbytes(1, E, H, 8) + qbytes(1, 1, H, 8)
        step_bytes = w_bytes + H * 2 + 2 * H * 2   # + x read, residual read/write
        # algorithmic bytes of each of the three launches: weights + activations read and
        # results written (router logits/candidates and ids/probs are a few hundred bytes)
        stage_bytes = {
            "decode_router_shared": qbytes(1, E, H, 8) + qbytes(1, 1, H, 8) + 2 * qbytes(1, I, H, 8) + H * 2
                                    + E * 4 + I * 4,
            "decode_experts_gate_up": 16 * qbytes(1, I, H, 8) + H * 2 + 8 * I * 4,
            "decode_down_merge": 9 * qbytes(1, H, I, 8) + 9 * I * 4 + 2 * H * 2,
        }
        stages = {}
        for name, (tot, cnt) in prof.items():
            avg = tot / max(cnt, 1)
            stages[name] = {"avg_us": avg * 1e3, "bytes": stage_bytes.get(name),
                            "GB_s": stage_bytes.get(name, 0) / (avg * 1e-3) / 1e9 if avg > 0 else None}
        self.free(built)
        return {"ms_per_step": ms, "bytes_per_step": step_bytes, "GB_s": step_bytes / (ms * 1e-3) / 1e9,
                "stages": stages}

    def decode_timeline(self, steps, layers=24):
        """Config 2 decode step with the decode kernels' in-kernel clock stamps (library built
        with `make timeline`): `steps` steps over `layers` rotating layer copies are captured in
        one HIP graph and replayed; the stamps hold the last step. Per kernel and stamp point the
        percentiles over all stamped waves, in us from the first wave entry of that step's router
        kernel; launch gaps = next kernel's first wave entry - previous kernel's last wave end."""
        import ctypes
        import numpy as np
        torch, dh = self.torch, self.dh
        L = dh.load()
        L.dih_decode_timeline_read.argtypes = [ctypes.c_void_p, ctypes.c_int]
        khz = L.dih_decode_timeline_clock_khz()
        if khz <= 0:
            raise RuntimeError("wall clock rate unavailable")
        built = [self.moe_layer(8) for _ in range(layers)]
        xs = self.bf16(64, H)
        res = self.bf16(H)
        dh.moe_decode(self.dev, built[0][1], xs[0], res)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            with torch.cuda.graph(g, stream=stream):
                for i in range(steps):
                    dh.moe_decode(self.dev, built[i % layers][1], xs[i % 64], res)
        torch.cuda.synchronize()
        for _ in range(2):
            g.replay()
        torch.cuda.synchronize()
        reps = []
        nb, nw, npnt = 512, 16, 4
        for _ in range(3):
            if L.dih_decode_timeline_clear() != 0:
                raise RuntimeError("timeline clear failed")
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            g.replay()
            torch.cuda.synchronize()
            wall = (time.perf_counter() - t0) * 1e3 / steps
            buf = np.zeros(3 * nb * nw * npnt, dtype=np.uint64)
            if L.dih_decode_timeline_read(buf.ctypes.data, buf.size) != 0:
                raise RuntimeError("timeline read failed")
            reps.append((buf.reshape(3, nb * nw, npnt).astype(np.int64), wall))
        del g
        self.free(built)
        us = 1e3 / khz
        names = ["decode_router_shared", "decode_experts_gate_up", "decode_down_merge"]
        points = [["entry", "x staged", "weights arrived + dot", "end"],
                  ["entry", "ranked, weights requested", "weights arrived + dot", "end"],
                  ["entry", "weights requested", "weights arrived + dot", "end"]]
        out = {"clock_khz": khz, "steps": steps, "layers": layers, "replays": []}
        for T, wall in reps:
            start = T[0][T[0][:, 0] > 0][:, 0].min()
            rep = {"graph_us_per_step": wall * 1e3, "kernels": {}}
            bounds = []
            for k, name in enumerate(names):
                t = T[k][(T[k][:, 0] > 0) & (T[k][:, 3] > 0)]
                kd = {"waves": int(len(t))}
                for j, pn in enumerate(points[k]):
                    col = t[:, j][t[:, j] > 0]
                    v = np.sort((col - start) * us)
                    kd[pn] = {"p10": round(float(v[len(v) // 10]), 2), "p50": round(float(v[len(v) // 2]), 2),
                              "p90": round(float(v[int(len(v) * 0.9)]), 2), "max": round(float(v[-1]), 2),
                              "min": round(float(v[0]), 2)}
                rep["kernels"][name] = kd
                bounds.append(((t[:, 0].min() - start) * us, (t[:, 3].max() - start) * us))
            rep["launch_gaps_us"] = {f"{names[k]} -> {names[k + 1]}": round(float(bounds[k + 1][0] - bounds[k][1]), 2)
                                     for k in range(2)}
            rep["step_us_first_entry_to_last_end"] = round(float(bounds[2][1] - bounds[0][0]), 2)
            out["replays"].append(rep)
        return out

    def qmv(self, steps, warmup, copies=64):
        """Config 1: one 8-bit [4096 x 2048] GEMV, bf16 in/out, rotating 64 weight copies."""
        torch, dh = self.torch, self.dh
        log(f"[qmv] building {copies} copies of 4096x2048 8-bit")
        ms_ = [self.matrix(1, 4096, 2048, 8) for _ in range(copies)]
        x = self.bf16(2048)
        y = torch.zeros(4096, dtype=torch.bfloat16, device="cuda")

        def step(i):
            dh.qmv(self.dev, ms_[i % copies], x, y, y_dtype=dh.BF16)

        ms, prof = self.timed_graph(step, steps, warmup)
        b = qbytes(1, 4096, 2048, 8) + 2048 * 2 + 4096 * 2
        tot, cnt = prof.get("qmv", (0.0, 1))
        kern = tot / max(cnt, 1)
        for m in ms_:
            m.dispose()
        return {"ms_per_step": ms, "bytes": b, "GB_s": b / (ms * 1e-3) / 1e9, "kernel_avg_us": kern * 1e3,
                "kernel_GB_s": b / (kern * 1e-3) / 1e9 if kern > 0 else None}

    def zipf_logits(self, T, s=1.1):
        torch = self.torch
        p = torch.arange(1, E + 1, dtype=torch.float64, device="cuda") ** -s
        p = p / p.sum()
        perm = torch.randperm(E, device="cuda", generator=self.gen)
        u = torch.rand((T, E), dtype=torch.float64, device="cuda", generator=self.gen).clamp_(1e-12, 1 - 1e-12)
        gumbel = -torch.log(-torch.log(u))
        return (torch.log(p)[perm][None, :] + gumbel).to(torch.bfloat16)

    def prefill(self, steps, warmup, T=512, bits=8, routing="zipf", layers=2):
        """Configs 3/4: grouped prefill MoE chunk over `layers` rotating layer copies."""
        torch, dh = self.torch, self.dh
        log(f"[prefill] T={T} bits={bits} routing={routing}: building {layers} layers")
        built = [self.moe_layer(bits, with_router=False) for _ in range(layers)]
        x = self.bf16(T, H)
        logits = self.zipf_logits(T) if routing == "zipf" else self.bf16(T, E)
        res = self.bf16(T, H)
        ids = torch.zeros((T, 8), dtype=torch.int32, device="cuda")
        dh.moe_prefill(self.dev, built[0][1], T, x, logits, res, trace=dh.make_trace(ids=ids))
        torch.cuda.synchronize()
        counts = torch.bincount(ids.reshape(-1).long(), minlength=E)
        touched = int((counts > 0).sum().item())

        def step(i):
            dh.moe_prefill(self.dev, built[i % layers][1], T, x, logits, res)

        ms, prof = self.timed_graph(step, steps, warmup)
        expert_w = 2 * qbytes(1, I, H, bits) + qbytes(1, H, I, bits)
        w_bytes = (touched + 1) * expert_w + qbytes(1, 1, H, 8)
        act_bytes = T * H * 2 * 3 + T * E * 2          # x read, residual read+write, logits
        flops_routed = 2.0 * T * 8 * (2 * I * H + H * I)
        flops_shared = 2.0 * T * (2 * I * H + H * I)
        flops = flops_routed + flops_shared
        stages = {}
        for name, (tot, cnt) in prof.items():
            stages[name] = {"avg_us": tot / max(cnt, 1) * 1e3}
        def stage_ms(name):
            tot, cnt = prof.get(name, (0, 1))
            return tot / max(cnt, 1)
        # (with the shared expert's launches on the library's side stream, config 4's
        # gate/up interval covers the routed launch and the down interval the rest up to the
        # join, so these per-stage rates are approximate there; ms_per_step is not affected)
        gu_ms = stage_ms("prefill_gate_up")
        dn_ms = stage_ms("prefill_down")
        gu_bytes = (touched + 1) * 2 * qbytes(1, I, H, bits)
        dn_bytes = (touched + 1) * qbytes(1, H, I, bits)
        if gu_ms > 0:
            stages.setdefault("prefill_gate_up", {"avg_us": 0.0})
            stages["prefill_gate_up"].update(avg_us=gu_ms * 1e3,
                bytes=gu_bytes, GB_s=gu_bytes / (gu_ms * 1e-3) / 1e9,
                TFLOP_s=(2.0 / 3.0) * flops / (gu_ms * 1e-3) / 1e12)
        if dn_ms > 0:
            stages.setdefault("prefill_down", {"avg_us": 0.0})
            stages["prefill_down"].update(avg_us=dn_ms * 1e3,
                bytes=dn_bytes, GB_s=dn_bytes / (dn_ms * 1e-3) / 1e9,
                TFLOP_s=(1.0 / 3.0) * flops / (dn_ms * 1e-3) / 1e12)
        self.free(built)
        tf = flops / (ms * 1e-3) / 1e12
        return {"tokens": T, "bits": bits, "routing": routing, "experts_touched": touched,
                "max_routes_per_expert": int(counts.max().item()), "ms_per_step": ms,
                "weight_bytes": w_bytes, "GB_s": (w_bytes + act_bytes) / (ms * 1e-3) / 1e9,
                "GFLOP": flops / 1e9, "TFLOP_s": tf, "mfma_frac": tf / PEAK_BF16_TFLOPS,
                "hbm_frac": (w_bytes + act_bytes) / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS,
                "tok_s_per_layer": T / (ms * 1e-3), "stages": stages}

    def dense(self, steps, warmup, T=4096):
        """Config 5: dense 8-bit projections at a 4096-token chunk."""
        torch, dh = self.torch, self.dh
        shapes = {"q_gate": (8192, 2048), "k": (512, 2048), "v": (512, 2048), "o": (2048, 4096),
                  "in_proj": (12288, 2048)}
        out = {}
        for name, (R, C) in shapes.items():
            m = self.matrix(1, R, C, 8)
            x = self.bf16(T, C)
            y = torch.zeros((T, R), dtype=torch.bfloat16, device="cuda")

            def step(i, m=m, x=x, y=y, T=T):
                dh.dense(self.dev, m, T, x, y, y_dtype=dh.BF16)

            ms, prof = self.timed_graph(step, max(2, steps // 4), min(warmup, 3))
            # the fused tile ("dense_qmm"), or the dequantization pass and the bf16 GEMM
            stage_ms = {k: tot / max(cnt, 1) for k, (tot, cnt) in prof.items() if k.startswith("dense")}
            kern = sum(stage_ms.values())
            flops = 2.0 * T * R * C
            out[name] = {"rows": R, "cols": C, "ms": ms, "TFLOP_s": flops / (ms * 1e-3) / 1e12,
                         "mfma_frac": flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
                         "kernel_avg_us": kern * 1e3,
                         "stages_us": {k: v * 1e3 for k, v in stage_ms.items()}}
            m.dispose()
            del x, y
        tot_f = sum(2.0 * T * r * c for r, c in shapes.values())
        tot_ms = sum(v["ms"] for v in out.values())
        return {"tokens": T, "per_matrix": out, "TFLOP_s": tot_f / (tot_ms * 1e-3) / 1e12,
                "mfma_frac": tot_f / (tot_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS}

    def dense_small(self, steps, warmup, copies=16):
        """Dense projection at short chunks (the GEMV-vs-GEMM dispatch policy of p_gemv,
        gpu_prefill.mm:603-620): q/gate [8192 x 2048] 8-bit at T = 1..64, weights rotated
        over `copies` (285 MB, beyond the MALL). Times dih_dense and, for comparison, the
        batched GEMV (dih_qmv over T <= 8 slots of expert 0)."""
        torch, dh = self.torch, self.dh
        R, C = 8192, 2048
        mats = [self.matrix(1, R, C, 8) for _ in range(copies)]
        out = {}
        for T in (1, 2, 4, 8, 16, 32, 64):
            x = self.bf16(T, C)
            y = torch.zeros((T, R), dtype=torch.bfloat16, device="cuda")
            ids = torch.zeros(T, dtype=torch.int32, device="cuda")
            res = {}
            for path in (("dense", "qmv") if T <= 8 else ("dense",)):
                def step(i, x=x, y=y, T=T, path=path):
                    m = mats[i % copies]
                    if path == "dense":
                        dh.dense(self.dev, m, T, x, y, y_dtype=dh.BF16)
                    else:
                        dh.qmv(self.dev, m, x, y, experts=ids if T > 1 else None, count=T, batched=True,
                               y_dtype=dh.BF16)
                ms, _ = self.timed_graph(step, max(8, steps // 2), min(warmup, 4))
                res[path] = {"us": ms * 1e3, "GB_s": qbytes(1, R, C, 8) / (ms * 1e-3) / 1e9}
            out[T] = res
            del x, y
        for m in mats:
            m.dispose()
        return out

    def attention(self, steps, warmup):
        """Full-attention layer (prefill_attention_bf16 + combine; p_fused_attention,
        gpu_prefill.mm:552-570): 16 query heads over 2 KV heads, head dim 256, bf16 cache.
        Cases: a 2048-token chunk on an empty cache, the last 2048-token chunk of a 32K
        prompt, and one decode token at 32K, all at the reference's default 1024-key rounding
        partition, plus the decode token with 32-key rounding (the decode kernel alone).
        FLOPs count the causal work only: 1024 per (query row, visible key) (q.k and p.v,
        2 x 256 multiply-adds)."""
        torch, dh = self.torch, self.dh
        out = {}
        for name, position, T, part in (("chunk2048_pos0", 0, 2048, 0), ("chunk2048_pos30720", 30720, 2048, 0),
                                        ("decode_pos32767", 32767, 1, 0), ("decode_pos32767_round32", 32767, 1, 32)):
            cap = position + T
            g = torch.Generator(device="cuda").manual_seed(5)
            keys = (torch.rand((cap, 512), device="cuda", generator=g) * 0.8 - 0.4).to(torch.bfloat16)
            vals = (torch.rand((cap, 512), device="cuda", generator=g) * 0.8 - 0.4).to(torch.bfloat16)
            q = torch.rand((T, 4096), device="cuda", generator=g) * 0.8 - 0.4
            raw = torch.rand((T, 8192), device="cuda", generator=g) * 4 - 2
            y = torch.zeros((T, 4096), device="cuda")

            def step(i, q=q, keys=keys, vals=vals, raw=raw, y=y, position=position, T=T, part=part):
                dh.attention(self.dev, q, keys, vals, raw, y, position, T, partition=part)

            n = max(4, steps // 12) if T > 1 else max(16, steps)
            ms, prof = self.timed_graph(step, n, min(warmup, 3))
            tot, cnt = prof.get("attention", (0, 1))
            ctot, ccnt = prof.get("attention_combine", (0, 1))
            stot, scnt = prof.get("attention_scores", (0, 1))
            visible = T * position + T * (T + 1) // 2
            flops = 1024.0 * 16 * visible
            kv_bytes = 2 * cap * 512 * 2
            out[name] = {"position": position, "tokens": T, "partition": dh.attention_partition(position, T, part),
                         "scores_avg_us": stot / max(scnt, 1) * 1e3,
                         "ms": ms, "GFLOP": flops / 1e9, "TFLOP_s": flops / (ms * 1e-3) / 1e12,
                         "mfma_frac": flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
                         "kv_GB_s": kv_bytes / (ms * 1e-3) / 1e9, "attn_kernel_avg_us": tot / max(cnt, 1) * 1e3,
                         "combine_avg_us": ctot / max(ccnt, 1) * 1e3}
            del keys, vals, q, raw, y
        return out

    def delta(self, steps, warmup):
        """Gated delta rule of one linear-attention layer (p_delta, gpu_prefill.mm:540-551):
        32 value heads x 128 rows x 128 key dims of f32 state, for a 2048-token chunk
        (chunkwise), a 63-token chunk (sequential, the longest below the switch) and one
        decode token. FLOPs count the recurrence's own work, 4 x 2 x 128 x 128 per head and
        token (decay, prediction, update, readout)."""
        torch, dh = self.torch, self.dh
        out = {}
        cases = [("chunk2048", 2048, 0), ("chunk2048_sequential", 2048, 1), ("chunk63", 63, 0),
                 ("chunk63_chunkwise", 63, 2), ("decode1", 1, 0)]
        if getattr(self.args, "delta_sweep", False):
            cases += [(f"chunk{T}_{p}", T, i) for T in (32, 40, 48, 56, 64, 96, 128, 256, 512, 1024)
                      for i, p in ((1, "sequential"), (2, "chunkwise"))]
        for name, T, path in cases:
            g = torch.Generator(device="cuda").manual_seed(7)
            conv = torch.randn((T, 8192), device="cuda", generator=g) * 0.1
            k = conv[:, 2048:4096].view(T, 16, 128)
            k /= k.norm(dim=2, keepdim=True)
            a = torch.rand((T, 32), device="cuda", generator=g) * 0.1 + 0.9
            b = torch.rand((T, 32), device="cuda", generator=g)
            raw = torch.randn((T, 8192), device="cuda", generator=g)
            state = torch.randn((32, 128, 128), device="cuda", generator=g) * 0.01
            hist = torch.zeros((3, 8192), device="cuda")
            y = torch.zeros((T, 4096), device="cuda")

            def step(i, conv=conv, a=a, b=b, raw=raw, state=state, hist=hist, y=y, T=T, path=path):
                dh.delta_rule(self.dev, state, hist, conv, a, b, raw, y, T, path=path)

            n = max(8, steps // 8) if T > 1 else max(16, steps)
            ms, prof = self.timed_graph(step, n, min(warmup, 3))
            flops = 8.0 * 128 * 128 * 32 * T
            stages = {k2: {"avg_us": v[0] / max(v[1], 1) * 1e3, "launches": v[1]} for k2, v in prof.items()}
            out[name] = {"tokens": T, "path": ["auto", "sequential", "chunkwise"][path], "ms": ms, "us_per_token": ms * 1e3 / T, "GFLOP": flops / 1e9,
                         "TFLOP_s": flops / (ms * 1e-3) / 1e12, "stages": stages}
            del conv, a, b, raw, state, hist, y
        return out

    def lm_head(self, steps, warmup, copies=2):
        """Config 5b: lm_head [248320 x 2048] 8-bit in 4 vocab slices, f32 logits, argmax."""
        torch, dh = self.torch, self.dh
        log(f"[lm_head] building {copies} copies of 4 x 62080 x 2048 8-bit")
        sets = [[self.matrix(1, 62080, 2048, 8) for _ in range(4)] for _ in range(copies)]
        x = self.bf16(2048)
        logits = torch.zeros(248320, dtype=torch.float32, device="cuda")
        nxt = torch.zeros(1, dtype=torch.int32, device="cuda")

        def step(i):
            dh.lm_head(self.dev, sets[i % copies], x, logits, nxt)

        ms, prof = self.timed_graph(step, max(2, steps // 4), min(warmup, 3))
        b = qbytes(1, 248320, 2048, 8) + 2048 * 2 + 248320 * 4
        tot, cnt = prof.get("lm_head_qmv", (0, 1))
        kern = tot / max(cnt, 1)
        for s in sets:
            for m in s:
                m.dispose()
        return {"ms_per_step": ms, "bytes": b, "GB_s": b / (ms * 1e-3) / 1e9,
                "qmv_kernel_avg_us": kern * 1e3,
                "qmv_kernel_GB_s": (b - 248320 * 4) / (kern * 1e-3) / 1e9 if kern > 0 else None}

    def copycal(self, steps, mbytes=512):
        """A plain device copy of known size: the reference point that scales rocprofv3's
        FETCH_SIZE / WRITE_SIZE counters to bytes."""
        torch = self.torch
        n = mbytes << 20
        a = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
        b = torch.empty_like(a)
        for _ in range(steps):
            b.copy_(a)
        torch.cuda.synchronize()
        return {"bytes_read_per_copy": n, "bytes_written_per_copy": n, "copies": steps}

    def peaks(self, read_gib=4, reps=5):
        """On-box ceilings (lib/libdih_peaks.so): a streaming read of `read_gib` GiB (well
        above the 256 MB MALL) and a register-resident bf16 MFMA loop, each swept over a few
        grid sizes; every point is the median of `reps` launches timed with HIP events on the
        stream the kernels run on. The best point of each sweep is the measured ceiling."""
        import ctypes
        import statistics
        torch = self.torch
        lib = ctypes.CDLL(os.path.join(ROOT, "infer.net_amd", "lib", "libdih_peaks.so"))
        lib.dihp_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int,
                                         ctypes.c_void_p]
        lib.dihp_mfma_loop.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                                       ctypes.c_void_p]
        lib.dihp_mfma_loop_flops.restype = ctypes.c_double
        lib.dihp_mfma_loop_flops.argtypes = [ctypes.c_int, ctypes.c_int]
        lib.dihp_stream_read_pieces.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p]
        lib.dihp_stream_read_pieces_blocks.restype = ctypes.c_size_t
        lib.dihp_stream_read_pieces_blocks.argtypes = [ctypes.c_size_t]
        stream = torch.cuda.current_stream()
        h = ctypes.c_void_p(stream.cuda_stream)

        def timed(launch):
            launch()
            ms = []
            for _ in range(reps):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                launch()
                e1.record(stream)
                e1.synchronize()
                ms.append(e0.elapsed_time(e1))
            return statistics.median(ms)

        nbytes = read_gib << 30
        buf = torch.empty(nbytes // 4, dtype=torch.int32, device="cuda").fill_(0x5a5a5a5a)
        sink = torch.empty(1 << 16, dtype=torch.int32, device="cuda")
        read = {}
        for blocks in (2048, 4096, 8192, 16384):
            def launch(blocks=blocks):
                rc = lib.dihp_stream_read(ctypes.c_void_p(buf.data_ptr()), nbytes, ctypes.c_void_p(sink.data_ptr()),
                                          blocks, h)
                assert rc == 0, rc
            read[blocks] = nbytes / (timed(launch) * 1e-3) / 1e9
        nb = int(lib.dihp_stream_read_pieces_blocks(nbytes))
        sink2 = torch.empty(nb, dtype=torch.int32, device="cuda")

        def launch_pieces():
            rc = lib.dihp_stream_read_pieces(ctypes.c_void_p(buf.data_ptr()), nbytes, ctypes.c_void_p(sink2.data_ptr()), h)
            assert rc == 0, rc
        read["pieces"] = nbytes / (timed(launch_pieces) * 1e-3) / 1e9
        del buf, sink2
        ops = torch.full((64 * 8,), 0x3F80, dtype=torch.int16, device="cuda")  # bf16 1.0
        iters = 2048
        mfma = {}
        for blocks in (1024, 2048, 4096):
            out = torch.empty(blocks * lib.dihp_mfma_threads(), dtype=torch.float32, device="cuda")

            def launch(blocks=blocks, out=out):
                rc = lib.dihp_mfma_loop(ctypes.c_void_p(ops.data_ptr()), iters, ctypes.c_void_p(out.data_ptr()),
                                        blocks, h)
                assert rc == 0, rc
            mfma[blocks] = lib.dihp_mfma_loop_flops(iters, blocks) / (timed(launch) * 1e-3) / 1e12
            assert bool((out == 1024.0 * iters).all()), "MFMA probe returned a wrong sum"
        torch.cuda.empty_cache()
        return {"hbm_read_GB_s": max(read.values()), "mfma_bf16_TFLOP_s": max(mfma.values()),
                "read_sweep_GB_s": {str(k): round(v, 1) for k, v in read.items()},
                "mfma_sweep_TFLOP_s": {str(k): round(v, 1) for k, v in mfma.items()},
                "method": f"stream read of {read_gib} GiB (grid-stride dwordx4 with 4 loads in flight per lane over "
                          f"2K-16K blocks, and one-shot 32 KB blocks of non-temporal loads, 8 in flight per lane) and "
                          f"{iters} rounds x 4 independent v_mfma_f32_32x32x16_bf16 per wave; median of "
                          f"{reps} launches per grid size, best grid size reported"}

    def load(self, reps=3):
        """Checkpoint loading (dih_checkpoint_moe_layer): one config-2 MoE layer written in the
        MLX safetensors layout to a temporary directory (so the shard files sit in the page
        cache), then loaded `reps` times into device matrices. Reports file -> HBM GB/s."""
        import shutil
        import tempfile
        import numpy as np
        sys.path.insert(0, ROOT)
        from tests import ckpt_util as cu
        dh = self.dh
        rng = np.random.default_rng(0)
        d = tempfile.mkdtemp(prefix="dih-load-")
        try:
            p = "language_model.model.layers.0."
            spec = [("mlp.gate", 1, E, H, 8), ("mlp.switch_mlp.gate_proj", E, I, H, 8),
                    ("mlp.switch_mlp.up_proj", E, I, H, 8), ("mlp.switch_mlp.down_proj", E, H, I, 8),
                    ("mlp.shared_expert.gate_proj", 1, I, H, 8), ("mlp.shared_expert.up_proj", 1, I, H, 8),
                    ("mlp.shared_expert.down_proj", 1, H, I, 8), ("mlp.shared_expert_gate", 1, 1, H, 8)]
            t, total = {}, 0
            for name, e, r, c, bits in spec:
                lead = () if e == 1 else (e,)
                w = rng.integers(0, 1 << 32, size=lead + (r, c * bits // 32), dtype=np.uint32)
                sc = np.full(lead + (r, c // 64), 0x3a80, dtype=np.uint16)
                bi = np.full(lead + (r, c // 64), 0xbf00, dtype=np.uint16)
                t.update(cu.matrix_tensors(p + name, w, sc, bi))
                total += w.nbytes + sc.nbytes + bi.nbytes
            cu.write_checkpoint(d, t, bits=8, shards=2)
            del t
            times = []
            for _ in range(reps + 1):
                t0 = time.perf_counter()
                with dh.Checkpoint(d) as ck:
                    _, mats = ck.moe_layer(self.dev, 0)
                times.append(time.perf_counter() - t0)
                for m in mats:
                    m.dispose()
            best = min(times[1:])
            return {"bytes": total, "ms": best * 1e3, "GB_s": total / best / 1e9,
                    "note": "shard files in the page cache; pread -> 2x64 MiB pinned staging -> H2D"}
        finally:
            shutil.rmtree(d, ignore_errors=True)

    def free(self, built):
        for mats, _ in built:
            for m in mats.values():
                if m is not None:
                    m.dispose()
        self.keep = [k for k in self.keep if all(k is not b[0] for b in built)]
        self.torch.cuda.empty_cache()


def host_description():
    """CPU model, the cores this process may run on, and the machine's logical CPU count."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "nproc": len(os.sched_getaffinity(0)), "logical_cpus": os.cpu_count()}


def cpu_baseline(seconds, runs=5):
    """The reference's CPU dequant-then-matmul path (oracle/oracle.c restatement of
    MatVec.cs:40-55 + quantized.mm:384-397, composed per Qwen36Model.cs:218-262) timed for
    config 2 on this host in two legs: single-threaded, as the reference runs it, and on
    every core this process may use (rows and experts split across OpenMP threads, at most
    16: the box's CPU share). Each leg does one warm-up step, then `runs` timed runs of the
    same number of steps; the reported figure is the median run. `value` is the all-cores
    leg, the stronger of the two baselines."""
    import statistics
    import numpy as np
    sys.path.insert(0, ROOT)
    from oracle import oracle as orc
    rng = np.random.default_rng(0)
    L = orc.MoeLayer(orc.random_matrix(rng, 1, E, H, 8, 1.25e-4, 5e-4), orc.random_matrix(rng, E, I, H, 8),
                     orc.random_matrix(rng, E, I, H, 8), orc.random_matrix(rng, E, H, I, 8),
                     orc.random_matrix(rng, 1, I, H, 8), orc.random_matrix(rng, 1, I, H, 8),
                     orc.random_matrix(rng, 1, H, I, 8), orc.random_matrix(rng, 1, 1, H, 8))
    xs = orc.round_bf16(rng.normal(size=(16, H)).astype(np.float32))
    b = 9 * (2 * qbytes(1, I, H, 8) + qbytes(1, H, I, 8)) + qbytes(1, E, H, 8) + qbytes(1, 1, H, 8) + 6 * H
    host = host_description()
    all_threads = max(1, min(16, host["nproc"]))

    def leg(threads, budget):
        t0 = time.perf_counter()
        orc.cpu_moe_token(L, xs[0], threads=threads)  # warm-up
        one = max(time.perf_counter() - t0, 1e-5)
        per_run = max(1, int(budget / runs / one))
        per_step = []
        n = 0
        for _ in range(runs):
            t0 = time.perf_counter()
            for _ in range(per_run):
                orc.cpu_moe_token(L, xs[n % 16], threads=threads)
                n += 1
            per_step.append((time.perf_counter() - t0) / per_run)
        dt = statistics.median(per_step)
        return {"GB_s": b / dt / 1e9, "ms_per_step": dt * 1e3, "threads": threads, "runs": runs,
                "steps_per_run": per_run, "run_ms_per_step": [round(t * 1e3, 3) for t in per_step]}

    single = leg(1, 0.6 * seconds)
    multi = leg(all_threads, 0.4 * seconds) if all_threads > 1 else single
    return {"value": multi["GB_s"], "unit": "GB/s", "cores": all_threads, "kind": "port",
            "sample": f"decode MoE steps (config 2, one 8-bit layer): 1 warm-up + median of {runs} runs "
                      f"of {multi['steps_per_run']} steps on {all_threads} threads "
                      f"({multi['ms_per_step']:.2f} ms/step); single-thread leg {single['GB_s']:.2f} GB/s "
                      f"over {runs} runs of {single['steps_per_run']} steps; oracle/oracle.c orc_cpu_moe_token",
            "ms_per_step": multi["ms_per_step"], "all_cores": multi, "single_thread": single, "host": host}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=240)
    ap.add_argument("--warmup", type=int, default=24)
    ap.add_argument("--workload", default="all")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--delta-sweep", action="store_true", help="delta: both paths at 32..1024 tokens")
    ap.add_argument("--layers", type=int, default=24,
                    help="decode: rotating layer copies (24 x 855 MB keeps every step's weights out of the 256 MB MALL)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); this build has no multi-GPU path.",
              file=sys.stderr)
        sys.exit(2)
    if int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py runs as a single process on one GPU.", file=sys.stderr)
        sys.exit(2)
    steps, warmup = max(1, args.steps), max(0, args.warmup)
    wls = set(args.workload.split(","))
    if "decode_timeline" in wls:
        # the measurement build of the library (make -C infer.net_amd timeline), loaded in
        # place of the product library before anything else loads it
        import deepinfer_hip as dh
        dh.LIB_PATH = os.path.join(os.path.dirname(dh.LIB_PATH), "libdeepinfer_hip_timeline.so")
        b = Bench(args)
        print(json.dumps({"decode_timeline": b.decode_timeline(min(steps, 48), layers=args.layers)}), flush=True)
        return
    b = Bench(args)
    on = lambda name: "all" in wls or name in wls  # noqa: E731
    res = {}
    if on("decode"):
        res["decode"] = b.decode(steps, warmup, layers=args.layers)
        log(f"[decode] {res['decode']['GB_s']:.0f} GB/s, {res['decode']['ms_per_step'] * 1e3:.2f} us/step")
    if on("qmv"):
        res["qmv"] = b.qmv(steps, warmup)
        log(f"[qmv] {res['qmv']['GB_s']:.0f} GB/s")
    if on("prefill"):
        res["prefill"] = b.prefill(max(2, steps // 12), min(warmup, 3))
        log(f"[prefill] {res['prefill']['TFLOP_s']:.1f} TFLOP/s, {res['prefill']['GB_s']:.0f} GB/s")
    if on("prefill5"):
        res["prefill5"] = b.prefill(max(2, steps // 24), min(warmup, 2), T=2048, bits=5, routing="uniform")
        log(f"[prefill5] {res['prefill5']['TFLOP_s']:.1f} TFLOP/s, {res['prefill5']['GB_s']:.0f} GB/s")
    if on("dense"):
        res["dense"] = b.dense(steps, warmup)
        log(f"[dense] {res['dense']['TFLOP_s']:.1f} TFLOP/s")
    if on("attention"):
        res["attention"] = b.attention(steps, warmup)
        for name, r in res["attention"].items():
            log(f"[attention] {name}: {r['ms'] * 1e3:.1f} us, {r['TFLOP_s']:.1f} TFLOP/s, KV {r['kv_GB_s']:.0f} GB/s")
    if on("delta"):
        res["delta"] = b.delta(steps, warmup)
        for name, r in res["delta"].items():
            log(f"[delta] {name}: {r['ms'] * 1e3:.1f} us ({r['us_per_token']:.2f} us/token), {r['TFLOP_s']:.2f} TFLOP/s")
    if "load" in wls:
        res["load"] = b.load()
        log(f"[load] {res['load']['GB_s']:.1f} GB/s ({res['load']['bytes'] / 1e6:.0f} MB in {res['load']['ms']:.1f} ms)")
    if "dense_small" in wls:
        res["dense_small"] = b.dense_small(steps, warmup)
        for T, r in res["dense_small"].items():
            q = f", batched qmv {r['qmv']['us']:.1f} us" if "qmv" in r else ""
            log(f"[dense_small] T={T}: dense {r['dense']['us']:.1f} us{q}")
    if "copycal" in wls:
        print(json.dumps(b.copycal(max(1, min(steps, 8)))), flush=True)
        return
    if on("lm_head"):
        res["lm_head"] = b.lm_head(steps, warmup)
        log(f"[lm_head] {res['lm_head']['GB_s']:.0f} GB/s")
    if on("peaks"):
        res["peaks"] = b.peaks()
        log(f"[peaks] HBM read {res['peaks']['hbm_read_GB_s']:.0f} GB/s, "
            f"bf16 MFMA {res['peaks']['mfma_bf16_TFLOP_s']:.0f} TFLOP/s")

    if "decode" in res:
        d = res["decode"]
        head = {"metric": metric_name(), "value": d["GB_s"], "unit": "GB/s", "ms_per_step": d["ms_per_step"],
                "dtype": "f32", "percent_of_peak": 100.0 * d["GB_s"] / PEAK_HBM_GBS,
                "config": {"workload": "decode MoE step (BASELINE config 2): 1 token, 8-bit g64, 256 experts "
                                       "top-8, hidden 2048, intermediate 512, shared expert + sigmoid gate, "
                                       "router GEMV, weighted sum into a bf16 residual; 24 rotating layer copies",
                           "bytes_per_step": d["bytes_per_step"], "layers_rotated": 24}}
        roof = None
        if d["stages"]:
            dom = max(d["stages"].items(), key=lambda kv: kv[1]["avg_us"])
            roof = {"kernel": dom[0], "bound": "hbm", "achieved": dom[1]["GB_s"], "peak": PEAK_HBM_GBS,
                    "unit": "GB/s", "frac": dom[1]["GB_s"] / PEAK_HBM_GBS if dom[1]["GB_s"] else None,
                    "traffic": traffic_from_profiles(dom[0]), "avg_us": dom[1]["avg_us"],
                    "bytes_per_launch": dom[1]["bytes"]}
            if "peaks" in res and dom[1]["GB_s"]:
                roof["measured_peak"] = res["peaks"]["hbm_read_GB_s"]
                roof["frac_of_measured_peak"] = dom[1]["GB_s"] / res["peaks"]["hbm_read_GB_s"]
            # every decode kernel's fraction: from this run's HIP events, and from the average
            # duration the committed rocprofv3 kernel trace of the same command measured
            kern = {}
            for name, st in d["stages"].items():
                rp = rocprof_avg_us_from_profiles(name)
                kern[name] = {"avg_us": st["avg_us"], "bytes": st["bytes"],
                              "frac": st["GB_s"] / PEAK_HBM_GBS if st["GB_s"] else None,
                              "rocprof_avg_us": rp,
                              "frac_rocprof": st["bytes"] / (rp * 1e3) / PEAK_HBM_GBS if rp and st["bytes"] else None}
            roof["kernels"] = kern
            roof["frac_rocprof"] = kern[dom[0]]["frac_rocprof"]
    else:
        k, v = next(iter(res.items()))
        if k == "attention":
            v = v["chunk2048_pos30720"]
        elif k == "delta":
            v = v["chunk2048"]
        head = {"metric": metric_name(), "value": v.get("GB_s") or v.get("TFLOP_s"),
                "unit": "GB/s" if "GB_s" in v else "TFLOP/s", "ms_per_step": v.get("ms_per_step", v.get("ms")),
                "dtype": "bf16" if k in ("prefill", "prefill5", "dense") else "f32", "config": {"workload": k}}
        roof = None
    tok = None
    if "decode" in res and "lm_head" in res:
        per_token_ms = 40 * res["decode"]["ms_per_step"] + res["lm_head"]["ms_per_step"]
        tok = {"decode_path_tok_s": 1e3 / per_token_ms,
               "note": "kernel-sum of this path only (40 MoE layers + lm_head), not model throughput"}
    cpu = None
    if not args.no_cpu and on("decode"):
        log(f"[cpu] timing the CPU baseline for ~{args.cpu_seconds:.0f} s")
        cpu = cpu_baseline(args.cpu_seconds)
    line = {"metric": head["metric"], "value": head["value"], "unit": head["unit"], "n_gpus": 1,
            "steps": steps, "warmup": warmup, "ms_per_step": head["ms_per_step"], "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": head["dtype"], "data": "synthetic",
            "config": head["config"], "roofline": roof, "cpu_baseline": cpu, "tok_s": tok,
            "peaks_measured": res.get("peaks"),
            "secondary": {k: v for k, v in res.items() if k not in ("decode", "peaks")}}
    if "decode" in res:
        line["secondary"]["decode_stages"] = res["decode"]["stages"]
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
