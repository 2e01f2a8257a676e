"""Benchmark: paged GQA decode attention (Llama-3-8B shape) and stick relayout
on one MI355X.  Prints one JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]

Workload (a "step"): one decode-attention call for batch 32, 32 q heads /
8 KV heads, head_dim 128, context 4096 per sequence, fp16 K/V ~ N(0,1) in
64-token stick-layout pages, block table a seeded permutation of the page
pool, split 512 tokens per wavefront (a whole sequence per workgroup, so the
call is one kernel).  Inputs are resident in HBM before the timed region;
two KV caches (1.07 GB) alternate so the 256 MB last-level cache cannot
serve a step from the previous one.

Also timed: under "more_configs", the dense MHA decode call (q [1, 8, 1, 64], k/v
[1, 8, 512, 64]; absolute µs, launch-bound; eager, and prepared once as SdpaCall), the
Llama-3-8B decode step through SDPA with dense K/V (q [32, 32, 1, 128], k/v [32, 8, 4096,
128]), its batch-1 (absolute µs) and long-context (q [4, 64, 1, 128], k/v [4, 8, 32768, 128])
counterparts, head_dim 64 decode through SDPA (q [32, 16, 1, 64] against k/v [32, 16, 2048,
64], and the same bytes as q [16, 16, 1, 64] against [16, 16, 4096, 64]), a chunked prefill
(q [4, 32, 128, 128] against k/v [4, 8, 4096, 128]), the ragged batch (64 sequences, context
~ U[128, 32768], seeded), the long-context step (batch 4, 64 q / 8 KV heads, append one
token at position 131072, attend over 131073 tokens) and prefill SDPA, causal, full and
with an fp16 / boolean [4096, 4096] mask (batch 1, 32 q / 8 KV heads, 4096 tokens), and for
reference torch's fp16 [8192, 8192] GEMM (the MFMA rate a plain library GEMM reaches on the
same device); under "relayout", fp16 [4096, 4096] -> sticks, sticks -> row-major and
transpose-restick, rotating 9 buffer pairs (576 MiB), torch's copy and the identity copy
through the same 128 KiB tile pattern, with torch's CPU view/permute/contiguous of the same
closed forms as its CPU baseline, and a KV cache of 8 sequences [8, 8, 2048, 128] to and
from its default layout.

Timing: HIP events on the stream the kernels are launched on, around K
back-to-back steps, after W warm-up steps.  GB/s = algorithmic bytes / time.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "decode-attn µs/step + achieved HBM GB/s (% peak); relayout GB/s"
PEAK_HBM_GBS = 8000.0
# HBM bytes per decode_split_list_kernel launch at split 512, from rocprofv3
# --pmc FETCH_SIZE and WRITE_SIZE (KiB per dispatch) scaled by the same
# counters on torch's 32 MiB device copy (x1.99860 and x1.0): 536.99 MB read
# + 0.26 MB written (profiles/decode_attention_llama3_8b_b32_ctx4096_hbm_counters.md).
# Re-measure both together whenever decode_split_list_kernel changes.
TRAFFIC_BYTES = 537_251_143
B, HQ, HKV, D, CTX, PAGE, SPLIT = 32, 32, 8, 128, 4096, 64, 512


def attn_bytes(B, Hq, Hkv, D, ctx_total, pages_total):
    """Algorithmic HBM bytes of one decode step: K+V once, q, out, block
    table, context lengths (split partials are not counted)."""
    return ctx_total * Hkv * D * 2 * 2 + 2 * B * Hq * D * 2 + 4 * pages_total + 4 * B


def timed(fn, steps, warmup, stream):
    import torch

    for _ in range(warmup):
        fn(0)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(steps):
        fn(i)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps  # per call
    print(f"bench: {steps} calls timed, {ms * 1e3:.2f} us each", file=sys.stderr, flush=True)  # progress
    return ms


def cpu_model() -> str:
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name"):
                return line.split(":", 1)[1].strip()
    except Exception:
        pass
    return "unknown"


def cpu_baseline(k_log_pages, v_log_pages, table, q, budget_s=12.0):
    """The reference's CPU path: torch CPU eager fp32 SDPA over gathered pages
    (oracle.attention), timed on the host cores for a bounded sample."""
    import torch

    from oracle import attention as OA

    torch.set_num_threads(os.cpu_count() or 1)
    nthreads = torch.get_num_threads()
    qs = q.float()
    done_seq = 0
    t0 = time.perf_counter()
    t_sdpa = 0.0
    while time.perf_counter() - t0 < budget_s:
        b = done_seq % q.shape[0]
        kb, vb = OA.gather_sequence(k_log_pages, v_log_pages, table[b], CTX)
        kt = torch.from_numpy(kb).float()[None]
        vt = torch.from_numpy(vb).float()[None]
        s0 = time.perf_counter()
        OA.sdpa_cpu_fp32(qs[b][None, :, None, :], kt, vt, scale=1 / math.sqrt(D))
        t_sdpa += time.perf_counter() - s0
        done_seq += 1
    elapsed = time.perf_counter() - t0
    seq_bytes = attn_bytes(1, HQ, HKV, D, CTX, CTX // PAGE)
    return {
        "value": round(seq_bytes * done_seq / elapsed / 1e9, 3),
        "unit": "GB/s",
        "cores": nthreads,
        "kind": "port",
        "sample": f"{done_seq} of the workload's sequences (page gather + torch CPU fp32 SDPA), "
                  f"{elapsed:.1f} s; SDPA alone {seq_bytes * done_seq / t_sdpa / 1e9:.3f} GB/s; "
                  f"os.cpu_count()={os.cpu_count()}, cpu={cpu_model()}",
        "us_per_step_equiv": round(elapsed / done_seq * B * 1e6, 1),
    }


def cpu_relayout_baseline(x, budget_s=1.0):
    """The relayout closed forms (to sticks: x.view(R, C/64, 64).permute(1, 0, 2); from sticks:
    the inverse; transpose-restick: x.view(R/64, 64, C).permute(0, 2, 1)) made contiguous by torch
    on the host cores, each repeated for about budget_s."""
    import torch

    torch.set_num_threads(os.cpu_count() or 1)
    R, C = x.shape
    sticks = x.view(R, C // 64, 64).permute(1, 0, 2).contiguous()
    ops = {
        "to_sticks": lambda: x.view(R, C // 64, 64).permute(1, 0, 2).contiguous(),
        "from_sticks": lambda: sticks.permute(1, 0, 2).reshape(R, C).contiguous(),
        "transpose_restick": lambda: x.view(R // 64, 64, C).permute(0, 2, 1).contiguous(),
    }
    res = {}
    nbytes = 2 * x.numel() * x.element_size()
    for name, fn in ops.items():
        n, t0 = 0, time.perf_counter()
        while n < 3 or time.perf_counter() - t0 < budget_s:
            fn()
            n += 1
        dt = (time.perf_counter() - t0) / n
        res[name] = {"us": round(dt * 1e6, 1), "GB/s": round(nbytes / dt / 1e9, 2)}
    res["cores"] = torch.get_num_threads()
    res["kind"] = "port"
    res["sample"] = f"fp16 [{R}, {C}] bit patterns, each op repeated for ~{budget_s:.0f} s; cpu={cpu_model()}"
    return res


def more_configs(tsa, dev, stream, steps, warmup, seed):
    """The dense decode call, the ragged batch, the long-context append +
    attend step and prefill SDPA, timed the same way (the two paged caches
    are far larger than the last-level cache)."""
    import torch

    res = {}
    g = torch.Generator().manual_seed(seed)
    gg = torch.Generator(device=dev).manual_seed(seed + 1)

    # dense MHA decode: q [1, 8, 1, 64], k/v [1, 8, 512, 64], scale 1/8 (launch-bound:
    # absolute µs; one short-decode kernel, a block per head)
    q1 = torch.randn((1, 8, 1, 64), generator=gg, device=dev).half()
    k1 = torch.randn((1, 8, 512, 64), generator=gg, device=dev).half()
    v1 = torch.randn((1, 8, 512, 64), generator=gg, device=dev).half()
    ms = timed(lambda i: tsa.sdpa_decode(q1, k1, v1, scale=0.125), steps, warmup, stream)
    call1 = tsa.SdpaCall(q1, k1, v1, scale=0.125)  # validated once, as a serving loop holds it
    ms_p = timed(lambda i: call1(), steps, warmup, stream)
    res["dense_mha_decode_b1_h8_s512_d64"] = {"us_per_call": round(ms * 1e3, 2),
                                               "us_per_call_prepared": round(ms_p * 1e3, 2),
                                               "algorithmic_bytes": 1_050_624, "kernels_per_step": 1}
    # the Llama-3-8B decode step through SDPA with dense (unpaged) K/V:
    # q [32, 32, 1, 128], k/v [32, 8, 4096, 128] (the split-KV decode kernel
    # on the dense K / V: one workgroup per (sequence, KV head))
    q2 = torch.randn((32, HQ, 1, D), generator=gg, device=dev).half()
    k2 = torch.randn((32, HKV, 4096, D), generator=gg, device=dev).half()
    v2 = torch.randn((32, HKV, 4096, D), generator=gg, device=dev).half()
    ms = timed(lambda i: tsa.scaled_dot_product_attention(q2, k2, v2, enable_gqa=True), steps, warmup, stream)
    nb = 2 * k2.numel() * 2 + 2 * q2.numel() * 2
    res["dense_gqa_decode_b32_h32_8_s4096"] = {
        "us_per_step": round(ms * 1e3, 2), "GB/s": round(nb / (ms * 1e-3) / 1e9, 1),
        "frac": round(nb / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4), "algorithmic_bytes": nb, "kernels_per_step": 1}
    del q2, k2, v2
    # batch-1 decode through SDPA with dense K/V: q [1, 32, 1, 128], k/v
    # [1, 8, 4096, 128] (keys split across blocks, the partials merged by the
    # last block in the same kernel)
    q4 = torch.randn((1, HQ, 1, D), generator=gg, device=dev).half()
    k4 = torch.randn((1, HKV, 4096, D), generator=gg, device=dev).half()
    v4 = torch.randn((1, HKV, 4096, D), generator=gg, device=dev).half()
    ms = timed(lambda i: tsa.scaled_dot_product_attention(q4, k4, v4, enable_gqa=True), steps, warmup, stream)
    call4 = tsa.SdpaCall(q4, k4, v4, enable_gqa=True)
    ms_p = timed(lambda i: call4(), steps, warmup, stream)
    res["dense_gqa_decode_b1_h32_8_s4096"] = {"us_per_call": round(ms * 1e3, 2),
                                              "us_per_call_prepared": round(ms_p * 1e3, 2), "kernels_per_step": 1}
    del q4, k4, v4
    # long-context decode through SDPA with dense K/V: q [4, 64, 1, 128],
    # k/v [4, 8, 32768, 128] (8 chunks per (sequence, KV head), their partials
    # merged by the last of them in the same kernel)
    q3 = torch.randn((4, 64, 1, D), generator=gg, device=dev).half()
    k3 = torch.randn((4, HKV, 32768, D), generator=gg, device=dev).half()
    v3 = torch.randn((4, HKV, 32768, D), generator=gg, device=dev).half()
    ws3 = torch.empty(max(1, tsa._lib.lib().spyre_sdpa_fwd_call_workspace_bytes(None, 0, None, 4, 64, HKV, 1, 32768, D)),
                      dtype=torch.uint8, device=dev)
    ms = timed(lambda i: tsa.scaled_dot_product_attention(q3, k3, v3, enable_gqa=True, workspace=ws3), steps, warmup,
               stream)
    nb = 2 * k3.numel() * 2 + 2 * q3.numel() * 2
    res["dense_gqa_decode_b4_h64_8_s32768"] = {
        "us_per_step": round(ms * 1e3, 2), "GB/s": round(nb / (ms * 1e-3) / 1e9, 1),
        "frac": round(nb / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4), "algorithmic_bytes": nb, "kernels_per_step": 1}
    del q3, k3, v3, ws3
    # head_dim 64 decode through SDPA: q [32, 16, 1, 64], k/v [32, 16, 2048, 64]
    # (two K/V sets, 537 MB, rotated)
    q5 = torch.randn((32, 16, 1, 64), generator=gg, device=dev).half()
    kv5 = [(torch.randn((32, 16, 2048, 64), generator=gg, device=dev).half(),
            torch.randn((32, 16, 2048, 64), generator=gg, device=dev).half()) for _ in range(2)]
    calls5 = [tsa.SdpaCall(q5, k, v) for k, v in kv5]
    ms = timed(lambda i: calls5[i & 1](), steps, warmup, stream)
    nb = 2 * kv5[0][0].numel() * 2 + 2 * q5.numel() * 2
    res["dense_mha_decode_b32_h16_s2048_d64"] = {
        "us_per_step": round(ms * 1e3, 2), "GB/s": round(nb / (ms * 1e-3) / 1e9, 1),
        "frac": round(nb / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4), "algorithmic_bytes": nb, "kernels_per_step": 1}
    del q5, kv5, calls5
    # the same bytes at D 64 in one round of workgroups: q [16, 16, 1, 64],
    # k/v [16, 16, 4096, 64] (256 (sequence, head) workgroups, 8 runs of 64
    # tokens per wavefront, against 512 workgroups of 4 runs above)
    q7 = torch.randn((16, 16, 1, 64), generator=gg, device=dev).half()
    kv7 = [(torch.randn((16, 16, 4096, 64), generator=gg, device=dev).half(),
            torch.randn((16, 16, 4096, 64), generator=gg, device=dev).half()) for _ in range(2)]
    calls7 = [tsa.SdpaCall(q7, k, v) for k, v in kv7]
    ms = timed(lambda i: calls7[i & 1](), steps, warmup, stream)
    nb = 2 * kv7[0][0].numel() * 2 + 2 * q7.numel() * 2
    res["dense_mha_decode_b16_h16_s4096_d64"] = {
        "us_per_step": round(ms * 1e3, 2), "GB/s": round(nb / (ms * 1e-3) / 1e9, 1),
        "frac": round(nb / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4), "algorithmic_bytes": nb, "kernels_per_step": 1}
    del q7, kv7, calls7
    # chunked prefill: q [4, 32, 128, 128] against k/v [4, 8, 4096, 128] (keys split
    # 8 ways so the blocks fill the device, partials merged)
    q6 = torch.randn((4, HQ, 128, D), generator=gg, device=dev).half()
    kv6 = [(torch.randn((4, HKV, 4096, D), generator=gg, device=dev).half(),
            torch.randn((4, HKV, 4096, D), generator=gg, device=dev).half()) for _ in range(2)]
    calls6 = [tsa.SdpaCall(q6, k, v, enable_gqa=True) for k, v in kv6]
    ms = timed(lambda i: calls6[i & 1](), steps, max(warmup, 25), stream)  # MFMA work: past the clock settling
    fl = 4.0 * 4 * HQ * 128 * 4096 * D
    res["chunked_prefill_b4_h32_8_q128_k4096"] = {
        "us_per_step": round(ms * 1e3, 2), "TFLOP/s": round(fl / (ms * 1e-3) / 1e12, 1),
        "frac_of_f16_mfma_peak": round(fl / (ms * 1e-3) / 2.5e15, 4), "flops": fl,
        "kernels_per_step": 2}
    del q6, kv6, calls6

    def paged(lens, Hq, Hkv):
        pages = [(c + PAGE - 1) // PAGE for c in lens]
        total = sum(pages)
        cache = tsa.PagedKVCache(total, Hkv, D, device=dev, zero=False)
        cache.k.normal_(generator=gg)
        cache.v.normal_(generator=gg)
        perm = torch.randperm(total, generator=g).to(torch.int32)
        table = torch.zeros((len(lens), max(pages)), dtype=torch.int32)
        k = 0
        for b, n in enumerate(pages):
            table[b, :n] = perm[k:k + n]
            k += n
        q = torch.randn((len(lens), Hq, D), generator=gg, device=dev).half()
        return cache, table.to(dev), q, total

    # ragged: 64 sequences, context ~ U[128, 32768]
    lens = torch.randint(128, 32769, (64,), generator=g).tolist()
    cache, table, q, total = paged(lens, HQ, HKV)
    lt = torch.tensor(lens, dtype=torch.int32, device=dev)
    call = tsa.PagedDecode(q, cache.k, cache.v, table, lt, split_tokens=SPLIT, max_context_len=max(lens))
    ms = timed(lambda i: call(), steps, warmup, stream)
    nb = attn_bytes(64, HQ, HKV, D, sum(lens), total)
    res["ragged_b64_ctx_u128_32768"] = {
        "us_per_step": round(ms * 1e3, 2), "GB/s": round(nb / (ms * 1e-3) / 1e9, 1),
        "frac": round(nb / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4), "algorithmic_bytes": nb,
        "sum_ctx": sum(lens), "kernels_per_step": call.passes}
    del cache, call

    # long context: batch 4, 64 q / 8 KV heads, append at 131072, attend 131073
    B5, HQ5, CTX5 = 4, 64, 131072
    cache, table, q, total = paged([CTX5 + 1] * B5, HQ5, HKV)
    lt = torch.full((B5,), CTX5 + 1, dtype=torch.int32, device=dev)
    pos = torch.full((B5,), CTX5, dtype=torch.int32, device=dev)
    k_new = torch.randn((B5, HKV, D), generator=gg, device=dev).half()
    v_new = torch.randn((B5, HKV, D), generator=gg, device=dev).half()
    call = tsa.PagedDecode(q, cache.k, cache.v, table, lt, split_tokens=SPLIT, max_context_len=CTX5 + 1)

    def step(i):
        tsa.kv_append(k_new, v_new, cache.k, cache.v, table, pos)
        call()

    ms = timed(step, steps, warmup, stream)
    nb = attn_bytes(B5, HQ5, HKV, D, B5 * (CTX5 + 1), total) + 2 * 2 * B5 * HKV * D * 2
    res["long_ctx_b4_g8_ctx131072_append"] = {
        "us_per_step": round(ms * 1e3, 2), "GB/s": round(nb / (ms * 1e-3) / 1e9, 1),
        "frac": round(nb / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4), "algorithmic_bytes": nb,
        "kernels_per_step": 1 + call.passes}
    del cache, call

    # prefill SDPA: batch 1, 32 q / 8 KV heads, 4096 tokens, causal and full
    # (MFMA-bound; flops count the unmasked score pairs only).  From a cold
    # start, back-to-back calls 6 .. ~25 run up to 30 % slower while the
    # power management settles, then return to the first calls' rate; each
    # configuration is timed after PREFILL_WARMUP calls.
    PREFILL_WARMUP = 25
    S, PEAK_F16 = 4096, 2.5e15
    q = torch.randn((1, HQ, S, D), generator=gg, device=dev).half()
    k = torch.randn((1, HKV, S, D), generator=gg, device=dev).half()
    v = torch.randn((1, HKV, S, D), generator=gg, device=dev).half()
    for causal in (True, False):
        ms = timed(lambda i: tsa.scaled_dot_product_attention(q, k, v, is_causal=causal, enable_gqa=True),
                   max(steps // 5, 10), PREFILL_WARMUP, stream)
        flops = 4 * HQ * D * (S * (S + 1) / 2 if causal else S * S)
        res["prefill_b1_h32_8_s4096" + ("_causal" if causal else "")] = {
            "us_per_step": round(ms * 1e3, 1), "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 1),
            "frac_of_f16_mfma_peak": round(flops / (ms * 1e-3) / PEAK_F16, 4), "flops": flops,
            "kernels_per_step": 1}
    # the same with a [4096, 4096] mask broadcast over heads: an fp16 bias
    # ~ N(0, 1) and a boolean keep-mask (70 % kept); every pair is computed
    ws = torch.empty(tsa.sdpa.workspace_bytes(1, HKV, S, D), dtype=torch.uint8, device=dev)
    masks = {"mask_f16": torch.randn((S, S), generator=gg, device=dev).half(),
             "mask_bool": torch.rand((S, S), generator=gg, device=dev) < 0.7}
    for name, m in masks.items():
        ms = timed(lambda i: tsa.scaled_dot_product_attention(q, k, v, attn_mask=m, enable_gqa=True, workspace=ws),
                   max(steps // 5, 10), PREFILL_WARMUP, stream)
        flops = 4 * HQ * D * S * S
        res["prefill_b1_h32_8_s4096_" + name] = {
            "us_per_step": round(ms * 1e3, 1), "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 1),
            "frac_of_f16_mfma_peak": round(flops / (ms * 1e-3) / PEAK_F16, 4), "flops": flops,
            "kernels_per_step": 1}
    del masks, ws
    # For reference, the MFMA rate a plain library GEMM reaches on the same
    # box: torch's fp16 [8192, 8192] x [8192, 8192] (hipBLASLt), timed the
    # same way after the same warm-up.
    n = 8192
    ga = torch.randn((n, n), generator=gg, device=dev).half()
    gb = torch.randn((n, n), generator=gg, device=dev).half()
    ms = timed(lambda i: torch.mm(ga, gb), max(steps // 5, 10), PREFILL_WARMUP, stream)
    flops = 2 * n ** 3
    res["torch_gemm_f16_8192_reference"] = {
        "us_per_step": round(ms * 1e3, 1), "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 1),
        "frac_of_f16_mfma_peak": round(flops / (ms * 1e-3) / PEAK_F16, 4), "flops": flops}
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--split", type=int, default=SPLIT, help="tokens per KV split (multiple of 64)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(this path has no multi-GPU component)", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import torch_spyre_amd as tsa

    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(dev)
    seed = 0xAFFE

    # ---------------- decode attention (the workload) ----------------
    n_pages = B * CTX // PAGE
    g = torch.Generator().manual_seed(seed)
    gg = torch.Generator(device=dev).manual_seed(seed)
    caches, tables = [], []
    for r in range(2):
        c = tsa.PagedKVCache(n_pages, HKV, D, device=dev, zero=False)
        c.k.normal_(generator=gg)
        c.v.normal_(generator=gg)
        caches.append(c)
        tables.append(torch.randperm(n_pages, generator=g).to(torch.int32).view(B, CTX // PAGE).to(dev))
    q = torch.randn((B, HQ, D), generator=gg, device=dev).half()
    lens = torch.full((B,), CTX, dtype=torch.int32, device=dev)
    split = args.split
    ws = torch.empty(tsa.workspace_bytes(B, HQ, HKV, D, CTX, split), dtype=torch.uint8, device=dev)
    out = torch.empty_like(q)

    # One step = one decode call (one kernel at this shape), timed back to
    # back.  When a split size makes the call two kernels, the split pass
    # (the dominant kernel) is also timed on its own for the roofline.
    calls = [tsa.PagedDecode(q, c.k, c.v, t, lens, split_tokens=split, max_context_len=CTX,
                             workspace=ws, out=out) for c, t in zip(caches, tables)]
    ms = timed(lambda i: calls[i & 1](), args.steps, args.warmup, stream)
    if calls[0].passes == 1:
        split_ms = ms
    else:
        split_ms = timed(lambda i: calls[i & 1].split(), args.steps, args.warmup, stream)
    nbytes = attn_bytes(B, HQ, HKV, D, B * CTX, n_pages)
    gbs = nbytes / (ms * 1e-3) / 1e9
    split_gbs = nbytes / (split_ms * 1e-3) / 1e9
    more = more_configs(tsa, dev, stream, min(args.steps, 50), min(args.warmup, 5), seed)

    # ---------------- relayout (config: [4096, 4096] fp16) ----------------
    R = C = 4096
    nbuf = 9  # 9 x (32 MiB in + 32 MiB out) > 512 MiB: a step's buffers are out of the 256 MB MALL

    def bits16(i):
        """Random 16-bit patterns; NaN/Inf exponents (0x7C00 all set) get their top exponent bit
        cleared."""
        u = torch.randint(0, 1 << 16, (R, C), device=dev, dtype=torch.int32,
                          generator=torch.Generator(device=dev).manual_seed(seed + 100 + i))
        u = torch.where((u & 0x7C00) == 0x7C00, u ^ 0x4000, u)
        return u.to(torch.int16).view(torch.float16)

    xs = [bits16(i) for i in range(nbuf)]
    dflt = tsa.SpyreTensorLayout([R, C], torch.float16)
    trl = tsa.transpose_restick_layout(R, C)
    devs = [tsa.device_buffer(tsa.to_device_layout(x, dflt)) for x in xs]
    outs_dev = [torch.empty_like(d) for d in devs]
    outs_host = [torch.empty_like(x) for x in xs]
    to_plan = tsa.dma_plan([R, C], [C, 1], [C, 1], 0, dflt, True)
    from_plan = tsa.dma_plan([R, C], [C, 1], [C, 1], 0, dflt, False)
    tr_plan = [tsa.restick_plan([R, C], dflt, trl)]
    rel_bytes = 2 * R * C * 2
    relayout = {}
    DmaCopy = tsa.relayout.DmaCopy
    for name, calls in (
        ("to_sticks", [DmaCopy(xs[i], outs_dev[i], to_plan) for i in range(nbuf)]),
        ("from_sticks", [DmaCopy(devs[i], outs_host[i], from_plan) for i in range(nbuf)]),
        ("transpose_restick", [DmaCopy(devs[i], outs_dev[i], tr_plan) for i in range(nbuf)]),
    ):
        t = timed(lambda i: calls[i % nbuf](), args.steps, args.warmup, stream)
        relayout[name] = {"us": round(t * 1e3, 3), "GB/s": round(rel_bytes / (t * 1e-3) / 1e9, 1),
                          "frac": round(rel_bytes / (t * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
    # plain device copies of the same bytes, for reference: torch's, and this
    # library's flat nest -- the relayouts' 128 KiB LDS tile pattern with the
    # identity mapping (dma_block_copy_kernel: 32 runs of 4 KiB, 8 KiB apart,
    # per workgroup, loads landed before the stores), the rate that pattern
    # itself sustains
    t = timed(lambda i: outs_host[i % nbuf].copy_(xs[i % nbuf]), args.steps, args.warmup, stream)
    relayout["torch_copy_reference"] = {"us": round(t * 1e3, 3), "GB/s": round(rel_bytes / (t * 1e-3) / 1e9, 1)}
    flat = [DmaCopy(xs[i], outs_host[i], tsa.relayout.flat_plan(R * C)) for i in range(nbuf)]
    t = timed(lambda i: flat[i % nbuf](), args.steps, args.warmup, stream)
    relayout["identity_tile_copy"] = {"us": round(t * 1e3, 3), "GB/s": round(rel_bytes / (t * 1e-3) / 1e9, 1),
                                      "frac": round(rel_bytes / (t * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
    del devs, outs_dev, outs_host, flat
    # a KV cache of 8 sequences, [8, 8, 2048, 128] fp16 (32 MiB), to and from its default layout
    # [8, 2048, 2, 8, 64]: the 8 sequences sit beside the stick (8 x 128 / 128 x 8 stick tiles)
    kv_size = [8, 8, 2048, 128]
    kv_st = [8 * 2048 * 128, 2048 * 128, 128, 1]
    kv_lay = tsa.SpyreTensorLayout(kv_size, torch.float16)
    kxs = [xb.view(kv_size) for xb in (bits16(i) for i in range(nbuf))]
    kdevs = [torch.empty(tsa.relayout.alloc_shape(kv_size, torch.float16, kv_lay), dtype=torch.float16, device=dev)
             for _ in range(nbuf)]
    kv = {}
    for name, calls in (
        ("to_sticks", [DmaCopy(kxs[i], kdevs[i], tsa.dma_plan(kv_size, kv_st, kv_st, 0, kv_lay, True))
                       for i in range(nbuf)]),
        ("from_sticks", [DmaCopy(kdevs[i], kxs[i], tsa.dma_plan(kv_size, kv_st, kv_st, 0, kv_lay, False))
                         for i in range(nbuf)]),
    ):
        t = timed(lambda i: calls[i % nbuf](), args.steps, args.warmup, stream)
        kv[name] = {"us": round(t * 1e3, 3), "GB/s": round(rel_bytes / (t * 1e-3) / 1e9, 1),
                    "frac": round(rel_bytes / (t * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
    relayout["kv_cache_b8_h8_s2048_d128"] = kv
    del kxs, kdevs

    result = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "us_per_step": round(ms * 1e3, 2),
        "frac_of_peak": round(gbs / PEAK_HBM_GBS, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "Llama-3-8B-shaped paged GQA decode attention",
                   "batch": B, "q_heads": HQ, "kv_heads": HKV, "head_dim": D, "context": CTX,
                   "page_tokens": PAGE, "split_tokens": split, "kv_dtype": "fp16"},
        "roofline": {"bound": "hbm", "achieved": round(split_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(split_gbs / PEAK_HBM_GBS, 4), "traffic": TRAFFIC_BYTES,
                     "kernel": "decode_split_list_kernel<128>", "kernel_us": round(split_ms * 1e3, 2),
                     "algorithmic_bytes": nbytes},
        "more_configs": more,
        "relayout": relayout,
    }

    if not args.no_cpu:
        c = caches[0]
        from oracle import attention as OA

        k_log, v_log = OA.pages_to_logical(c.k.cpu().numpy(), c.v.cpu().numpy(), n_pages, HKV, D)
        result["cpu_baseline"] = cpu_baseline(k_log, v_log, tables[0].cpu().numpy(), q.cpu())
        result["relayout"]["cpu_baseline"] = cpu_relayout_baseline(xs[0].cpu())
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
