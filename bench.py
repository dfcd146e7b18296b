"""Benchmark of the gfx950 GQA attention hot path (one JSON line on stdout).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--settle-s T] [--workloads ...]

A step is one pass of the attention hot path over one batch of synthetic,
seeded inputs already resident in HBM:
  prefill  K-Norm + RoPE row kernel (K-hat), then the fused prefill kernel
           (Q-Norm + RoPE on load, causal GQA FlashAttention forward);
  decode   append of the new token's K-hat/V into the cache, then the decode
           kernel (a persistent grid streaming the ragged cache) and its merge;
           the paged form fuses the append into the decode launch;
  chunk    a prompt continuation into a paged cache: the chunk's K-hat/V
           appended into its pages, then the paged prefill kernel over all
           keys so far through the block table (no dense copy).
The headline ``value`` is prefill TFLOP/s on the Qwen3-1.7B-like layer
(B8 S2048 Hq16 Hkv8 D128 causal bf16); FLOPs are the algorithmic
4*D*B*Hq*S(S+1)/2 (QK^T + PV over causal pairs).  ``roofline`` divides the
prefill kernel's own FLOPs by its average duration: K launches of it back to
back on its launch stream between two HIP events, after the K timed steps
(``ms_per_step``, with nothing between the launches).  ``secondary`` holds
the other workloads, each with its roofline (decode bytes
sum_b 2*Hkv*T_b*D*2 + 2*B*Hq*D*2; backward FLOPs 2.5x the forward's, the five
matrix products of FlashAttention-2; chunk FLOPs 4*D*B*Hq*(C*p0 + C(C+1)/2)
for C queries after p0 cached keys).
Before its W warmup and K timed steps, each workload runs its own step
untimed for ``--settle-s`` seconds (default 0.2): the GPU raises its clock over
the first ~40 ms of sustained load (the 1.7B-like step goes from ~0.20 to
~0.165 ms) and lowers it again after ~0.5 s idle, e.g. while a CPU baseline
runs, so without it the short workloads would be timed during the ramp.
``cpu_baseline`` (top level for the headline, inside each ``secondary`` entry
for the others) times the reference's own composition -- QK-Norm, RoPE,
repeat_interleave, SDPA, restated in the oracle -- in fp32 on the host cores, on
each workload's own inputs: C2/C3 and both backward shapes in full, the decode
as B=1 slices with their own lengths, C5 as one KV group of four (the
extrapolation stated in ``sample``).  A sample shorter than CPU_MIN_S is
repeated in whole passes (``passes``).
``cores`` is the number of threads torch used; ``host_cpu_count`` is
os.cpu_count().  ``roofline.traffic`` is profile-derived (``traffic_source``);
``roofline.traffic_ratio`` divides it by the kernel's compulsory HBM bytes
(prefill: Q, K, V in and O out; decode: the cache rows once, Q, O; backward:
Q, K, V, O, dO in and dQ, dK, dV out).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
METRIC = "prefill attn TFLOP/s (% bf16 MFMA peak); decode KV GB/s (% HBM peak)"
YARN = {"type": "yarn", "factor": 4.0, "original_max_position_embeddings": 32768}


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _randn(shape, seed, device, dtype=torch.bfloat16, cpu=True):
    if cpu:
        g = torch.Generator().manual_seed(seed)
        return torch.randn(*shape, generator=g).to(dtype).to(device)
    g = torch.Generator(device=device).manual_seed(seed)
    return torch.randn(*shape, generator=g, device=device, dtype=dtype)


class Prefill:
    kind = "prefill"

    def __init__(self, nq, name, B, S, Hq, Hkv, D, seed, rope_scaling=None, wscale=0.02,
                 device="cuda", cpu_gen=True):
        self.nq, self.name = nq, name
        self.B, self.S, self.Hq, self.Hkv, self.D = B, S, Hq, Hkv, D
        # projections' (B, S, H, D) storage viewed as (B, H, S, D), as in the model
        self.q = _randn((B, S, Hq, D), seed, device, cpu=cpu_gen).transpose(1, 2)
        self.k = _randn((B, S, Hkv, D), seed + 100, device, cpu=cpu_gen).transpose(1, 2)
        self.v = _randn((B, S, Hkv, D), seed + 200, device, cpu=cpu_gen).transpose(1, 2)
        g = torch.Generator().manual_seed(seed + 300)
        self.qw = (1 + wscale * torch.randn(D, generator=g)).to(device)
        self.kw = (1 + wscale * torch.randn(D, generator=g)).to(device)
        cos, sin = nq.build_tables(D, S, 1e6, rope_scaling)
        self.cos, self.sin = cos.to(device), sin.to(device)
        self.khat = torch.empty(B, S, Hkv, D, dtype=torch.bfloat16, device=device).transpose(1, 2)
        self.out = torch.empty(B, S, Hq, D, dtype=torch.bfloat16, device=device).transpose(1, 2)
        self.work = 4.0 * D * B * Hq * S * (S + 1) / 2
        # compulsory HBM bytes of the kernel: Q in and O out, K-hat and V in
        self.algo_bytes = 2 * B * S * (Hq + Hkv) * D * 2
        self.rope_scaling = rope_scaling

        # validated, pre-bound launches: one foreign call each per step
        self.k_call = nq.qk_norm_rope(k=self.k, k_out=self.khat, k_weight=self.kw, eps=1e-6,
                                      cos=self.cos, sin=self.sin, plan=True)
        self.p_call = nq.attention_prefill(self.q, self.khat, self.v, q_weight=self.qw, eps=1e-6,
                                           cos=self.cos, sin=self.sin, causal=True, out=self.out,
                                           plan=True)

    def step(self):
        self.k_call.launch()
        self.p_call.launch()

    def timed_launch(self):
        """The kernel the roofline is about (K-hat is unchanged between steps)."""
        self.p_call.launch()

    def describe(self):
        return {"workload": self.name, "batch": self.B, "seq_len": self.S, "num_heads": self.Hq,
                "num_kv_heads": self.Hkv, "head_dim": self.D, "causal": True,
                "rope": "yarn x4" if self.rope_scaling else "theta 1e6"}

    def roofline(self, kernel_ms, traffic=None):
        ach = self.work / (kernel_ms * 1e-3) / 1e12
        return {"bound": "mfma", "achieved": round(ach, 2), "peak": PEAK_BF16_TFLOPS,
                "unit": "TFLOP/s", "frac": round(ach / PEAK_BF16_TFLOPS, 4), "traffic": traffic,
                "kernel": "prefill_kernel", "kernel_ms": round(kernel_ms, 5)}

    def throughput(self, step_ms):
        return self.work / (step_ms * 1e-3) / 1e12, "TFLOP/s"


class Decode:
    kind = "decode"

    def __init__(self, nq, name, B, Hq, Hkv, D, Tcap, seed, device="cuda"):
        self.nq, self.name = nq, name
        self.B, self.Hq, self.Hkv, self.D, self.Tcap = B, Hq, Hkv, D, Tcap
        g = torch.Generator().manual_seed(seed)
        self.lens_cpu = torch.randint(1024, Tcap + 1, (B,), generator=g, dtype=torch.int32)
        self.lens = self.lens_cpu.to(device)
        self.row = (self.lens_cpu - 1).to(device)            # slot of the new token
        self.max_len = int(self.lens_cpu.max())
        gd = torch.Generator(device=device).manual_seed(seed)
        self.kc = torch.randn(B, Hkv, Tcap, D, generator=gd, device=device, dtype=torch.bfloat16)
        self.vc = torch.randn(B, Hkv, Tcap, D, generator=gd, device=device, dtype=torch.bfloat16)
        self.q = _randn((B, Hq, 1, D), seed + 1, device)
        self.knew = _randn((B, Hkv, 1, D), seed + 2, device)
        self.vnew = _randn((B, Hkv, 1, D), seed + 3, device)
        self.w = torch.ones(D, device=device)
        cos, sin = nq.build_tables(D, Tcap, 1e6)
        self.cos, self.sin = cos.to(device), sin.to(device)
        self.out = torch.empty(B, Hq, D, dtype=torch.bfloat16, device=device)
        nbytes = nq.decode_workspace_bytes(B, Hq, Hkv, D, self.max_len)
        self.ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)
        self.work = float(2 * Hkv * D * 2 * int(self.lens_cpu.sum()) + 2 * B * Hq * D * 2)
        self.algo_bytes = self.work

        self.a_call = nq.qk_norm_rope(k=self.knew, v=self.vnew, k_out=self.kc, v_out=self.vc,
                                      k_weight=self.w, eps=1e-6, cos=self.cos, sin=self.sin,
                                      pos_base=self.row, kv_row_base=self.row, plan=True)
        self.d_call = nq.attention_decode(self.q, self.kc, self.vc, self.lens, max_len=self.max_len,
                                          q_weight=self.w, eps=1e-6, cos=self.cos, sin=self.sin,
                                          out=self.out, workspace=self.ws, plan=True)

    def step(self):
        self.a_call.launch()
        self.d_call.launch()

    def timed_launch(self):
        """The decode kernel and its merge (the append writes the same rows every step)."""
        self.d_call.launch()

    def describe(self):
        return {"workload": self.name, "batch": self.B, "num_heads": self.Hq,
                "num_kv_heads": self.Hkv, "head_dim": self.D, "cache_capacity": self.Tcap,
                "kv_lens": "U[1024, %d], sum %d" % (self.Tcap, int(self.lens_cpu.sum()))}

    def roofline(self, kernel_ms, traffic=None):
        ach = self.work / (kernel_ms * 1e-3) / 1e9
        return {"bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(ach / PEAK_HBM_GBS, 4), "traffic": traffic,
                "kernel": "decode_stream_kernel + decode_merge_kernel", "kernel_ms": round(kernel_ms, 5)}

    def throughput(self, step_ms):
        return self.work / (step_ms * 1e-3) / 1e9, "GB/s"


class PagedDecode(Decode):
    """The same decode against a paged pool, with the append fused into the decode launch.

    64-row pages are dealt to the sequences in a seeded random order.  Sequence b holds
    lens[b] - 1 keys; the launch norms, rotates and writes the new token's K (and V) at row
    lens[b] - 1 and attends all lens[b] keys, so the bytes match the dense workload's.
    """

    def __init__(self, nq, name, B, Hq, Hkv, D, Tcap, seed, page=64, device="cuda"):
        self.nq, self.name, self.page = nq, name, page
        self.B, self.Hq, self.Hkv, self.D, self.Tcap = B, Hq, Hkv, D, Tcap
        g = torch.Generator().manual_seed(seed)
        self.lens_cpu = torch.randint(1024, Tcap + 1, (B,), generator=g, dtype=torch.int32)
        self.held = (self.lens_cpu - 1).to(device)           # keys before the new token
        self.lens_out = torch.empty(B, dtype=torch.int32, device=device)
        self.max_len = int(self.lens_cpu.max())
        npp = Tcap // page
        self.bt = torch.randperm(B * npp, generator=g).view(B, npp).to(torch.int32).to(device)
        gd = torch.Generator(device=device).manual_seed(seed)
        self.kp = torch.randn(B * npp, Hkv, page, D, generator=gd, device=device, dtype=torch.bfloat16)
        self.vp = torch.randn(B * npp, Hkv, page, D, generator=gd, device=device, dtype=torch.bfloat16)
        self.q = _randn((B, Hq, 1, D), seed + 1, device)
        self.knew = _randn((B, Hkv, 1, D), seed + 2, device)
        self.vnew = _randn((B, Hkv, 1, D), seed + 3, device)
        self.w = torch.ones(D, device=device)
        cos, sin = nq.build_tables(D, Tcap, 1e6)
        self.cos, self.sin = cos.to(device), sin.to(device)
        self.out = torch.empty(B, Hq, D, dtype=torch.bfloat16, device=device)
        nbytes = nq.decode_workspace_bytes(B, Hq, Hkv, D, self.max_len)
        self.ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)
        self.work = float(2 * Hkv * D * 2 * int(self.lens_cpu.sum()) + 2 * B * Hq * D * 2)
        self.algo_bytes = self.work
        self.d_call = nq.attention_decode_paged(
            self.q, self.kp, self.vp, self.bt, self.held, max_len=self.max_len, k_new=self.knew,
            v_new=self.vnew, k_weight=self.w, lens_out=self.lens_out, q_weight=self.w, eps=1e-6,
            cos=self.cos, sin=self.sin, out=self.out, workspace=self.ws, plan=True)

    def step(self):
        self.d_call.launch()

    def timed_launch(self):
        self.d_call.launch()

    def describe(self):
        d = super().describe()
        d["cache"] = f"paged, {self.page}-row pages in a seeded random order, append fused"
        return d


class PagedChunk:
    """One chunk of a chunked prefill into a paged cache: the last 2048 tokens of 8192-token
    sequences whose first 6144 keys already sit in 64-row pages dealt in a seeded random
    order.  A step appends the chunk's K-hat (norm and rotation fused) and V into its pages,
    then the chunk's queries attend all keys through the block table (causal, true
    positions)."""
    kind = "prefill"

    def __init__(self, nq, name, B, T, C, Hq, Hkv, D, seed, page=64, device="cuda"):
        self.nq, self.name, self.page = nq, name, page
        self.B, self.T, self.C, self.Hq, self.Hkv, self.D = B, T, C, Hq, Hkv, D
        self.p0 = T - C
        self.q = _randn((B, C, Hq, D), seed, device).transpose(1, 2)
        self.k = _randn((B, C, Hkv, D), seed + 100, device).transpose(1, 2)
        self.v = _randn((B, C, Hkv, D), seed + 200, device).transpose(1, 2)
        g = torch.Generator().manual_seed(seed + 300)
        self.qw = (1 + 0.02 * torch.randn(D, generator=g)).to(device)
        self.kw = (1 + 0.02 * torch.randn(D, generator=g)).to(device)
        cos, sin = nq.build_tables(D, T, 1e6)
        self.cos, self.sin = cos.to(device), sin.to(device)
        npp = T // page
        self.bt = torch.randperm(B * npp, generator=g).view(B, npp).to(torch.int32).to(device)
        # the cached rows: unit-rms keys (as K-hat is) and N(0,1) values
        gd = torch.Generator(device=device).manual_seed(seed + 400)
        kp = torch.randn(B * npp, Hkv, page, D, generator=gd, device=device)
        self.kp = (kp * torch.rsqrt(kp.pow(2).mean(-1, keepdim=True))).to(torch.bfloat16)
        self.vp = torch.randn(B * npp, Hkv, page, D, generator=gd, device=device, dtype=torch.bfloat16)
        self.out = torch.empty(B, C, Hq, D, dtype=torch.bfloat16, device=device).transpose(1, 2)
        self.work = 4.0 * D * B * Hq * (C * self.p0 + C * (C + 1) / 2)
        self.algo_bytes = 2 * B * C * Hq * D * 2 + 2 * B * T * Hkv * D * 2  # Q, O; all T keys' K-hat, V
        self.a_call = nq.kv_append_paged(self.k, self.v, self.kp, self.vp, self.bt, k_weight=self.kw,
                                         eps=1e-6, cos=self.cos, sin=self.sin, row_offset=self.p0,
                                         pos_offset=self.p0, plan=True)
        self.p_call = nq.attention_prefill_paged(self.q, self.kp, self.vp, self.bt, T=T, q_weight=self.qw,
                                                 eps=1e-6, cos=self.cos, sin=self.sin, causal=True,
                                                 pos_offset=self.p0, out=self.out, plan=True)

    def step(self):
        self.a_call.launch()
        self.p_call.launch()

    def timed_launch(self):
        """The paged prefill (the append rewrites the same rows every step)."""
        self.p_call.launch()

    def describe(self):
        return {"workload": self.name, "batch": self.B, "seq_len": self.T, "chunk": self.C,
                "cached_keys": self.p0, "num_heads": self.Hq, "num_kv_heads": self.Hkv,
                "head_dim": self.D, "causal": True, "rope": "theta 1e6",
                "cache": f"paged, {self.page}-row pages in a seeded random order"}

    def roofline(self, kernel_ms, traffic=None):
        ach = self.work / (kernel_ms * 1e-3) / 1e12
        return {"bound": "mfma", "achieved": round(ach, 2), "peak": PEAK_BF16_TFLOPS,
                "unit": "TFLOP/s", "frac": round(ach / PEAK_BF16_TFLOPS, 4), "traffic": traffic,
                "kernel": "prefill_kernel (paged)", "kernel_ms": round(kernel_ms, 5)}

    def throughput(self, step_ms):
        return self.work / (step_ms * 1e-3) / 1e12, "TFLOP/s"


class Backward:
    """FlashAttention-2 backward (dQ kernel, which also forms Delta, then dK/dV) of a causal prefill."""
    kind = "backward"

    def __init__(self, nq, name, B, S, Hq, Hkv, D, seed, device="cuda"):
        self.nq, self.name = nq, name
        self.B, self.S, self.Hq, self.Hkv, self.D = B, S, Hq, Hkv, D
        # the attention's operands after QK-Norm + RoPE as the training path holds them:
        # Q-hat and K-hat head-major (the row kernel's outputs), V and dO in the
        # projections' (B, S, H, D) storage
        self.q = _randn((B, S, Hq, D), seed, device).transpose(1, 2).contiguous()
        self.k = _randn((B, S, Hkv, D), seed + 100, device).transpose(1, 2).contiguous()
        self.v = _randn((B, S, Hkv, D), seed + 200, device).transpose(1, 2)
        self.do = _randn((B, S, Hq, D), seed + 400, device).transpose(1, 2)
        self.o, self.lse = nq.attention_prefill(self.q, self.k, self.v, causal=True, return_lse=True)
        # FlashAttention-2 convention: 5 matrix products over the causal pairs
        self.work = 2.5 * 4.0 * D * B * Hq * S * (S + 1) / 2
        # Q, O, dO in and dQ out; K, V in and dK, dV out
        self.algo_bytes = 4 * B * S * (Hq + Hkv) * D * 2
        self.call = nq.ops.attention_backward(self.q, self.k, self.v, self.o, self.do, self.lse,
                                              causal=True, plan=True)

    def step(self):
        self.call.launch()

    def timed_launch(self):
        self.call.launch()

    def describe(self):
        return {"workload": self.name, "batch": self.B, "seq_len": self.S, "num_heads": self.Hq,
                "num_kv_heads": self.Hkv, "head_dim": self.D, "causal": True}

    def roofline(self, kernel_ms, traffic=None):
        ach = self.work / (kernel_ms * 1e-3) / 1e12
        return {"bound": "mfma", "achieved": round(ach, 2), "peak": PEAK_BF16_TFLOPS,
                "unit": "TFLOP/s", "frac": round(ach / PEAK_BF16_TFLOPS, 4), "traffic": traffic,
                "kernel": "bwd_dq_kernel + bwd_dkdv_kernel",
                "kernel_ms": round(kernel_ms, 5)}

    def throughput(self, step_ms):
        return self.work / (step_ms * 1e-3) / 1e12, "TFLOP/s"


def measured_traffic():
    """Per-launch HBM bytes (fetch + write) of the dominant kernels, as measured by
    rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE and summarised in
    profiles/attention_kernels_hbm_traffic.txt (counters already scaled by the
    plain-copy calibration).  Returns {workload: bytes}; empty if absent."""
    path = os.path.join(ROOT, "profiles", "attention_kernels_hbm_traffic.txt")
    out = {}
    if not os.path.exists(path):
        return out
    for line in open(path):
        f = line.split()
        if len(f) != 6 or line.startswith("#") or f[0] == "kernel":
            continue
        kern, w, fetch_mb, write_mb = f[0], f[1], float(f[4]), float(f[5])
        if kern in ("prefill_kernel", "decode_stream_kernel", "decode_merge_kernel",
                    "bwd_dq_kernel", "bwd_dkdv_kernel"):
            out[w] = out.get(w, 0.0) + (fetch_mb + write_mb) * 1e6
    return {w: int(b) for w, b in out.items()}


def settle(w, seconds):
    """Untimed back-to-back steps for `seconds` (at least one): the GPU raises
    its clock over the first ~40 ms of sustained load and drops it again when
    idle, so a workload's W warmup and K timed steps follow its own settle."""
    t0 = time.perf_counter()
    w.step()
    torch.cuda.synchronize()
    first = time.perf_counter() - t0
    every = max(1, int(0.01 / max(first, 1e-6)))  # check the clock about every 10 ms
    n = 1
    while time.perf_counter() - t0 < seconds:
        for _ in range(every):
            w.step()
        n += every
        torch.cuda.synchronize()
    return n


def time_workload(w, steps, warmup):
    """Step time from `steps` back-to-back steps with nothing between their
    launches; then the timed kernel(s) alone, `steps` launches back to back on
    their launch stream between two HIP events, for their average duration.
    (An event recorded between two launches holds the next dispatch ~6 us on
    this GPU and lengthens the bracketed interval, so neither figure is taken
    with events between launches.)"""
    for _ in range(warmup):
        w.step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        w.step()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(steps):
        w.timed_launch()
    end.record()
    torch.cuda.synchronize()
    return wall_ms / steps, start.elapsed_time(end) / steps


def _host():
    """Host threads used by torch's CPU kernels and the machine's CPU counts."""
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count()
    return {"cores": torch.get_num_threads(), "host_cpu_count": os.cpu_count(),
            "affinity_cpus": affinity}


def _cpu(t):
    return t.detach().float().cpu().contiguous()


CPU_MIN_S = 8.0    # a CPU sample shorter than this is repeated in whole passes


def cpu_prefill(w, groups=None):
    """The reference's prefill composition (QK-Norm, RoPE, repeat_interleave, SDPA;
    model/attention.py:95-115) in fp32 on the host cores, on the workload's own
    inputs, one batch row at a time.  ``groups``: time only the first KV groups
    (each Hq/Hkv query heads with their KV head) and extrapolate."""
    from oracle import reference_path_sdpa
    B, S, Hq, Hkv, D = w.B, w.S, w.Hq, w.Hkv, w.D
    G = Hq // Hkv
    ng = Hkv if groups is None else groups
    cos, sin, qw, kw = _cpu(w.cos)[:S], _cpu(w.sin)[:S], _cpu(w.qw), _cpu(w.kw)
    pos = torch.arange(S)
    sw = min(S, 8192)                         # warm-up, untimed: row 0's first 8192 positions
    reference_path_sdpa(_cpu(w.q[:1, :ng * G, :sw]), _cpu(w.k[:1, :ng, :sw]), _cpu(w.v[:1, :ng, :sw]),
                        q_weight=qw, k_weight=kw, eps=1e-6, cos=cos, sin=sin, q_pos=pos[:sw])
    dt, passes = 0.0, 0
    while passes == 0 or dt < CPU_MIN_S:
        for b in range(B):
            q, k, v = _cpu(w.q[b:b + 1, :ng * G]), _cpu(w.k[b:b + 1, :ng]), _cpu(w.v[b:b + 1, :ng])
            t0 = time.perf_counter()
            reference_path_sdpa(q, k, v, q_weight=qw, k_weight=kw, eps=1e-6, cos=cos, sin=sin,
                                q_pos=pos, causal=True)
            dt += time.perf_counter() - t0
            del q, k, v
        passes += 1
    frac = ng / Hkv
    work = w.work * frac * passes
    out = {"value": round(work / dt / 1e12, 4), "unit": "TFLOP/s", **_host(), "kind": "port",
           "seconds": round(dt, 3), "passes": passes}
    if frac == 1.0:
        out["sample"] = (f"the full workload ({B} batch rows, one at a time) x{passes} passes, "
                         f"{dt:.1f} s, fp32; QK-Norm + RoPE + repeat_interleave + SDPA")
    else:
        per = dt / passes
        out["sample"] = (f"{ng} of {Hkv} KV groups ({ng * G} query heads x {S} rows, causal) x{passes} "
                         f"passes, fp32, {per:.1f} s per pass; the full workload extrapolates "
                         f"x{Hkv // ng} to {per * Hkv / ng:.1f} s at the same rate")
        out["extrapolated_full_seconds"] = round(per * Hkv / ng, 2)
    return out


def cpu_decode(w, budget_s=20.0):
    """The reference's decode step (QK-Norm + RoPE of the new token, KVCache
    concatenation, repeat_interleave, SDPA; model/attention.py:24-46, 95-115) in
    fp32 on the host cores, as B=1 slices with each sequence's own length, over
    the workload's own cache contents.  Bytes are counted as on the GPU."""
    from oracle import reference_decode_sdpa
    Hq, Hkv, D = w.Hq, w.Hkv, w.D
    cos, sin, one = _cpu(w.cos), _cpu(w.sin), torch.ones(D)
    reference_decode_sdpa(torch.randn(1, Hq, 1, D), torch.randn(1, Hkv, 1, D), torch.randn(1, Hkv, 1, D),
                          torch.randn(1, Hkv, 63, D), torch.randn(1, Hkv, 63, D), q_weight=one,
                          k_weight=one, eps=1e-6, cos=cos, sin=sin)
    dt, dt_gqa, nbytes, done = 0.0, 0.0, 0, 0
    order = [b % w.B for b in range(64 * w.B)]      # whole passes while short of CPU_MIN_S
    for b in order:
        T = int(w.lens_cpu[b])
        kc, vc = _cpu(w.kc[b:b + 1, :, :T - 1]), _cpu(w.vc[b:b + 1, :, :T - 1])
        q, kn, vn = _cpu(w.q[b:b + 1]), _cpu(w.knew[b:b + 1]), _cpu(w.vnew[b:b + 1])
        t0 = time.perf_counter()
        reference_decode_sdpa(q, kn, vn, kc, vc, q_weight=one, k_weight=one, eps=1e-6, cos=cos, sin=sin)
        t1 = time.perf_counter()
        reference_decode_sdpa(q, kn, vn, kc, vc, q_weight=one, k_weight=one, eps=1e-6, cos=cos, sin=sin,
                              repeat_kv=False)
        dt_gqa += time.perf_counter() - t1
        dt += t1 - t0
        nbytes += 2 * Hkv * T * D * 2 + 2 * Hq * D * 2
        done += 1
        del kc, vc
        if dt + dt_gqa > budget_s or (done % w.B == 0 and dt >= CPU_MIN_S):
            break
    return {"value": round(nbytes / dt / 1e9, 3), "unit": "GB/s", **_host(), "kind": "port",
            "seconds": round(dt, 3),
            "sample": f"{done} slices ({done / w.B:.2f} passes over the {w.B} sequences) as B=1 "
                      f"slices with their own lengths "
                      f"({nbytes / 1e9:.3f} GB of the workload's bf16 algorithmic bytes), fp32; "
                      "norm + RoPE of the new token, cache concatenation, repeat_interleave, SDPA",
            "value_sdpa_enable_gqa": round(nbytes / dt_gqa / 1e9, 3),
            "note": "value_sdpa_enable_gqa: the same slices with SDPA grouping the heads itself "
                    "instead of the reference's repeat_interleave copy of the cache"}


def cpu_backward(w, rows=None):
    """The reference's training composition of the attention core (repeat_interleave +
    SDPA, model/attention.py:105-115) under autograd in fp32 on the host cores: the
    forward runs untimed, the backward is timed, one batch row at a time."""
    import torch.nn.functional as F
    B, Hq, Hkv = w.B, w.Hq, w.Hkv
    G = Hq // Hkv
    nr = B if rows is None else rows
    dt, passes = 0.0, 0

    def one(b):
        q, k, v = (_cpu(t[b:b + 1]).requires_grad_(True) for t in (w.q, w.k, w.v))
        do = _cpu(w.do[b:b + 1])
        o = F.scaled_dot_product_attention(q, k.repeat_interleave(G, 1), v.repeat_interleave(G, 1),
                                           is_causal=True)
        t0 = time.perf_counter()
        o.backward(do)
        return time.perf_counter() - t0

    one(0)                                          # row 0 once more, untimed: warm-up
    while passes == 0 or dt < CPU_MIN_S:
        for b in range(nr):
            dt += one(b)
        passes += 1
    work = w.work * nr / B * passes
    out = {"value": round(work / dt / 1e12, 4), "unit": "TFLOP/s", **_host(), "kind": "port",
           "seconds": round(dt, 3), "passes": passes}
    if nr == B:
        out["sample"] = (f"the full workload ({B} batch rows, one at a time) x{passes} passes, "
                         f"{dt:.1f} s, fp32 autograd backward")
    else:
        out["sample"] = (f"{nr} of {B} batch rows, fp32 autograd backward, {dt:.1f} s; the full "
                         f"workload extrapolates x{B // nr} to {dt * B / nr:.1f} s at the same rate")
        out["extrapolated_full_seconds"] = round(dt * B / nr, 2)
    return out


def cpu_chunk(w):
    """The reference's composition of a prompt continuation (norm + RoPE of the chunk,
    KVCache concatenation after the cached rows, repeat_interleave, SDPA with the
    bottom-right causal mask) in fp32 on the host cores, over the workload's own
    inputs and cached rows (gathered from the pages), one batch row at a time."""
    from oracle import reference_chunk_sdpa
    B, P, p0 = w.B, w.page, w.p0
    cos, sin, qw, kw = _cpu(w.cos), _cpu(w.sin), _cpu(w.qw), _cpu(w.kw)
    pages = w.bt[:, :p0 // P].long()

    def cached(pool, b):
        return _cpu(pool[pages[b]].permute(1, 0, 2, 3).reshape(1, w.Hkv, p0, w.D))

    dt, passes = 0.0, 0
    while passes == 0 or dt < CPU_MIN_S:
        for b in range(B):
            kc, vc = cached(w.kp, b), cached(w.vp, b)
            q, k, v = _cpu(w.q[b:b + 1]), _cpu(w.k[b:b + 1]), _cpu(w.v[b:b + 1])
            t0 = time.perf_counter()
            reference_chunk_sdpa(q, k, v, kc, vc, q_weight=qw, k_weight=kw, eps=1e-6, cos=cos, sin=sin)
            dt += time.perf_counter() - t0
            del kc, vc
        passes += 1
    return {"value": round(w.work * passes / dt / 1e12, 4), "unit": "TFLOP/s", **_host(), "kind": "port",
            "seconds": round(dt, 3), "passes": passes,
            "sample": f"the full chunk ({B} batch rows, one at a time) x{passes} passes, {dt:.1f} s, fp32; "
                      "QK-Norm + RoPE of the chunk + cache concatenation + repeat_interleave + SDPA"}


def cpu_baseline(name, w):
    if name == "c3_chunk":
        return cpu_chunk(w)
    if name in ("c2", "c3"):
        return cpu_prefill(w)
    if name == "c5":
        return cpu_prefill(w, groups=1)
    if name == "c4":
        return cpu_decode(w)
    if name == "c2_bwd":
        return cpu_backward(w)
    if name == "c3_bwd":
        return cpu_backward(w)
    return None


TRAFFIC_SOURCE = ("rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE over this workload's kernels, in runs of "
                  "their own scaled by a plain-copy calibration: profiles/attention_kernels_hbm_traffic.txt "
                  "(profile-derived, not measured in this run)")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--settle-s", type=float, default=0.2,
                    help="untimed steps for this long before each workload's warmup (GPU clock ramp)")
    ap.add_argument("--workloads", default="c2,c3,c4,c4_paged,c5,c3_chunk,c2_bwd,c3_bwd",
                    help="comma list of c2 (headline), c3, c4, c4_paged, c5, c3_chunk, c2_bwd, c3_bwd")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB (3 times), for scaling "
                         "rocprofv3 FETCH_SIZE/WRITE_SIZE readings to bytes")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the attention hot path is built and measured on a "
              "single MI355X (no collectives); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.calibrate_copy:
        n = args.calibrate_copy * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes": n * 4, "reps": 3}), flush=True)
        return
    import nano_qwen_amd as nq
    dev = "cuda"
    props = torch.cuda.get_device_properties(0)
    log(f"device {props.name} {getattr(props, 'gcnArchName', '')} CUs={props.multi_processor_count}")
    names = [w.strip() for w in args.workloads.split(",") if w.strip()]
    if "c2" not in names:
        names.insert(0, "c2")

    def build(name):
        if name == "c2":
            return Prefill(nq, "Qwen3-1.7B-like attention prefill B8 S2048 Hq16 Hkv8 D128 causal bf16",
                           8, 2048, 16, 8, 128, seed=1001)
        if name == "c3":
            return Prefill(nq, "Qwen3-8B-like attention prefill B4 S8192 Hq32 Hkv8 D128 causal bf16, "
                           "fused QK-Norm+RoPE", 4, 8192, 32, 8, 128, seed=1002)
        if name == "c4":
            return Decode(nq, "Qwen3-235B-A22B decode B64 Hq64 Hkv4 D128, ragged KV cache bf16",
                          64, 64, 4, 128, 32768, seed=1003)
        if name == "c4_paged":
            return PagedDecode(nq, "Qwen3-235B-A22B decode B64 Hq64 Hkv4 D128, paged KV cache bf16, "
                               "fused K/V append", 64, 64, 4, 128, 32768, seed=1003)
        if name == "c5":
            return Prefill(nq, "YaRN long-context prefill B1 S131072 Hq32 Hkv4 D128 causal bf16",
                           1, 131072, 32, 4, 128, seed=1004, rope_scaling=YARN, cpu_gen=False)
        if name == "c3_chunk":
            return PagedChunk(nq, "Qwen3-8B-like chunked prefill into a paged cache: the last 2048-token "
                              "chunk of B4 x 8192, Hq32 Hkv8 D128, causal bf16", 4, 8192, 2048, 32, 8, 128,
                              seed=1007)
        if name == "c2_bwd":
            return Backward(nq, "Qwen3-1.7B-like attention backward B8 S2048 Hq16 Hkv8 D128 causal bf16",
                            8, 2048, 16, 8, 128, seed=1005)
        if name == "c3_bwd":
            return Backward(nq, "Qwen3-8B-like attention backward B4 S8192 Hq32 Hkv8 D128 causal bf16",
                            4, 8192, 32, 8, 128, seed=1006)
        raise SystemExit(f"unknown workload {name}")

    results, cpu = {}, {}
    for name in names:
        w = build(name)
        # C5 takes ~0.1 s a step: at least 5 timed steps, a bounded number
        steps = args.steps if name != "c5" else max(5, min(args.steps, 8))
        warm = args.warmup if name != "c5" else 1
        n_settle = settle(w, args.settle_s)
        log(f"{name}: {steps} timed steps after {warm} warmup ({n_settle} settle steps, "
            f"{args.settle_s} s)")
        step_ms, kern_ms = time_workload(w, steps, warm)
        val, unit = w.throughput(step_ms)
        results[name] = {"config": w.describe(), "value": round(val, 3), "unit": unit,
                         "ms_per_step": round(step_ms, 5), "steps": steps, "warmup": warm,
                         "settle_steps": n_settle,
                         "roofline": w.roofline(kern_ms), "_algo_bytes": w.algo_bytes}
        log(f"{name}: {step_ms:.4f} ms/step, kernel avg {kern_ms:.4f} ms, {val:.2f} {unit}")
        if not args.no_cpu_baseline:
            log(f"{name}: cpu baseline (the reference's composition in fp32 on the host cores)")
            cpu[name] = cpu_baseline(name, w)
            if cpu[name] is not None:
                log(f"{name}: cpu {cpu[name]['value']} {cpu[name]['unit']} in {cpu[name]['seconds']} s")
        del w
        torch.cuda.empty_cache()

    traffic = measured_traffic()
    for name, r in results.items():
        r["roofline"]["traffic"] = traffic.get(name)
        r["roofline"]["traffic_source"] = TRAFFIC_SOURCE if name in traffic else None
        # counter bytes over the kernel's compulsory bytes (1.0: every byte crosses HBM once)
        algo = r.pop("_algo_bytes")
        r["roofline"]["traffic_ratio"] = round(traffic[name] / algo, 2) if name in traffic else None
        if name == "c4_paged" and "c4" in cpu:
            r["cpu_baseline"] = dict(cpu["c4"], sample="the c4 sequences (the reference has no "
                                     "paged cache): " + cpu["c4"]["sample"])
        elif cpu.get(name) is not None:
            r["cpu_baseline"] = cpu[name]
    head = results.pop("c2")
    line = {
        "metric": METRIC, "value": head["value"], "unit": head["unit"], "n_gpus": 1,
        "steps": head["steps"], "warmup": head["warmup"], "ms_per_step": head["ms_per_step"],
        "settle_s": args.settle_s, "settle_steps": head["settle_steps"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) inputs, QK-Norm weights 1+0.02*N(0,1))",
        "config": head["config"], "roofline": head["roofline"],
    }
    for r in results.values():
        r.pop("warmup")
    line["secondary"] = results
    if "cpu_baseline" in head:
        line["cpu_baseline"] = head["cpu_baseline"]
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
