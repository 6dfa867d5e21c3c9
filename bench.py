#!/usr/bin/env python3
"""CARE-KV fused decode attention benchmark on one MI355X.

Default workload is BASELINE config 3 (Mistral-7B GQA decode): batch 64,
32 query / 8 kv heads, head_dim 128, 32768-token context in 16-token pages,
uniform INT3 g=32 base with int8 page scales, 3% store budget (1 K + 1 V slot
per page), top-256 joint read (128 K + 128 V budget), query-aware K score,
exact softmax renormalisation.  One step = one decode token through one
layer's attention for the whole batch (projections excluded).  Inputs are
resident in HBM before timing; the timed region is K launches of the fused
kernel bracketed by HIP events on the launch stream.

Prints one JSON line on stdout; progress goes to stderr.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(ROOT, "care-kv-sparse-residual-correction-for-low-bit-kv-cache-quantization_amd")
for _p in (ROOT, PKG_DIR):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PAPER_ENV = dict(CAREKV_STORE_POLICY="residual_kind_aware", CAREKV_PREFILL_RESIDUAL_KIND="both",
                 CAREKV_KSCORE_LIVE="1", CAREKV_SCORE_NORMALIZE="1", CAREKV_K_CORRECTION_MODE="exact",
                 CAREKV_K_CORRECTION_SCALE="0.1")

CONFIGS = {
    # name: B, Hq, Hkv, D, N, read_k, read_v, distribution, seed
    "c1": dict(B=1, Hq=32, Hkv=4, D=64, N=512, rk=32, rv=32, dist="outlier8", seed=1,
               workload="config1 TinyLlama decode B=1 32q/4kv D=64 N=512"),
    "c2": dict(B=16, Hq=32, Hkv=32, D=128, N=4096, rk=64, rv=64, dist="student_t", seed=2,
               workload="config2 Llama-2-7B decode B=16 32q/32kv D=128 N=4096"),
    "c3": dict(B=64, Hq=32, Hkv=8, D=128, N=32768, rk=128, rv=128, dist="outlier10", seed=3,
               workload="config3 Mistral-7B GQA decode B=64 32q/8kv D=128 N=32768"),
    # config 3 with the base its text names: KIVI-style INT2 (per-channel K,
    # per-token V), kept as the reference keeps it, fp16 K_hat / V_hat pages
    "c3kivi": dict(B=64, Hq=32, Hkv=8, D=128, N=32768, rk=128, rv=128, dist="outlier10", seed=3, kivi=2,
                   workload="config3 Mistral-7B GQA decode B=64 32q/8kv D=128 N=32768, KIVI-style INT2 base"),
    # the same KIVI-style INT2 base stored packed (CacheConfig.kivi_packed):
    # 2-bit prompt pages, per-channel K scales, per-token V scales; the same
    # K_hat / V_hat values as the side buffer
    "c3kivip": dict(B=64, Hq=32, Hkv=8, D=128, N=32768, rk=128, rv=128, dist="outlier10", seed=3, kivi=2,
                    packed=True, workload="config3 Mistral-7B GQA decode B=64 32q/8kv D=128 N=32768, "
                                          "KIVI-style INT2 base, packed pages"),
}


# BASELINE config 4 (prefill / append path at Llama-2-13B shape); `--config c4`
PREFILL_CONFIG = dict(B=4, H=40, D=128, T=8192, bits=3, seed=4,
                      workload="config4 Llama-2-13B prefill B=4 40q/40kv D=128 T=8192")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gen_kv(torch, spec, b, device):
    """Synthetic post-RoPE K/V (Hkv, N, D) fp16 for sequence b (generated on device)."""
    g = torch.Generator(device=device).manual_seed(spec["seed"] * 100003 + b)
    H, N, D = spec["Hkv"], spec["N"], spec["D"]
    K = torch.randn(H, N, D, generator=g, device=device)
    V = torch.randn(H, N, D, generator=g, device=device)
    if spec["dist"].startswith("outlier"):
        mult = float(spec["dist"][len("outlier"):])
        for h in range(H):
            ch = torch.randperm(D, generator=g, device=device)[:4]
            K[h][:, ch] *= mult
    elif spec["dist"] == "student_t":
        n_ch = max(1, round(0.02 * D))
        for X in (K, V):
            for h in range(H):
                ch = torch.randperm(D, generator=g, device=device)[:n_ch]
                z = torch.randn(N, n_ch, generator=g, device=device)
                chi = (torch.randn(3, N, n_ch, generator=g, device=device) ** 2).sum(0)
                X[h][:, ch] = 6.0 * z / torch.sqrt(chi / 3.0)
    return K.half(), V.half()


def algorithmic_bytes(spec, cfg, cache, diag_np):
    """Bytes one decode step must move (the roofline model), split into the
    streaming kernel's share and the rest.

    Streaming kernel (reads every page once): packed K+V codes, int8 group
    scales, fp16 page masters, valid/has_meta/slot tables, every stored K
    residual slot (the query-aware K score needs dS on all of them) with its
    scale, q.  Rest of the step: the page tables again for scoring (v_sq,
    v_err), the selected V residual slots (union over the GQA group) and
    the fp16 output.  Workspace traffic between the kernels is not counted."""
    B, Hq, Hkv, D, N = spec["B"], spec["Hq"], spec["Hkv"], spec["D"], spec["N"]
    bits, G, P = cfg.base_bits, D // 32, math.ceil(N / 16)
    grp = Hq // Hkv
    k_slots = (cache.k_slot[0, :, :B, :P] >= 0).sum().item()          # stored K slots (all b, kvh)
    if spec.get("packed"):  # 2-bit K and V codes, fp16 V scales per (row, group), fp16 K channel scales
        base = 2 * N * D * 2 / 8 + N * G * 2 + D * 2
    elif spec.get("kivi"):  # fp16 K_hat / V_hat rows, no scales
        base = 2 * N * D * 2
    else:                 # K + V codes, int8 scales, fp16 masters
        base = 2 * N * D * bits / 8 + 2 * N * G + 2 * P * 2
    per_bkv_stream = (base
                      + P * (4 + 1 + (G + 4) * 4)     # valid, has_meta, k_slot, v_slot
                      + grp * D * 2)                  # q
    stream = B * Hkv * per_bkv_stream + k_slots * (16 * 32 // 2 + 2)
    v_union = 0
    for b in range(B):
        for h in range(Hkv):
            s = set()
            for j in range(grp):
                for x in diag_np[b, h * grp + j]:
                    if x < 0:
                        break
                    if (int(x) >> 30) == 1:
                        s.add(int(x) & ((1 << 30) - 1))
            v_union += len(s)
    rest = B * Hkv * P * (4 + 4 * 2) + v_union * (4 * D // 2 + 2) + B * Hq * D * 2
    return float(stream), float(stream + rest), int(k_slots), int(v_union)


def copy_calibration(mib, steps):
    """Plain device-to-device copy of `mib` MiB (torch copy kernel): the
    reference kernel for scaling FETCH_SIZE / WRITE_SIZE counters and an
    achievable-bandwidth yardstick."""
    import torch
    dev = torch.device("cuda", 0)
    n = mib * 2**20 // 4
    src = torch.empty(n, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        dst.copy_(src)
    e1.record()
    e1.synchronize()
    ms = e0.elapsed_time(e1) / steps
    gbs = 2 * n * 4 / (ms * 1e-3) / 1e9
    print(json.dumps({"metric": "device copy GB/s (read+write)", "value": round(gbs, 1), "unit": "GB/s",
                      "bytes_read_per_launch": n * 4, "bytes_written_per_launch": n * 4, "steps": steps,
                      "ms_per_launch": round(ms, 4)}), flush=True)


def load_traffic(kernel, workload):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 PMC
    summary (profiles/<kernel>_<workload>_traffic.json), or None."""
    p = os.path.join(ROOT, "profiles", f"{kernel}_{workload}_traffic.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        return json.load(f)


def oracle_slice_from_device(cache, seq, kvh, spec):
    """Copy one (sequence, kv head) of the device cache into the CPU oracle."""
    from oracle.check import oracle_slice_from_device as copy_slice
    return copy_slice(cache, seq, kvh, num_heads=spec["Hq"] // spec["Hkv"], read_budget_mode="absolute",
                      read_abs_k=spec["rk"], read_abs_v=spec["rv"], route_policy="joint",
                      store_budget_mode="ratio", store_budget_ratio=0.03)


def slice_ids(spec, slices):
    """(sequence, kv head) pairs of the sampled slices, spread over both."""
    B, Hkv = spec["B"], spec["Hkv"]
    out, seen = [], set()
    for i in range(slices * 4):
        sk = ((i * 37) % B, (i * 5 + i // B) % Hkv)
        if sk not in seen:
            seen.add(sk)
            out.append(sk)
        if len(out) == slices:
            break
    return out


def cpu_baseline(cache, spec, q_np, slices, out_np=None, diag_np=None):
    """Time the oracle (numpy restatement of the reference decode path:
    read_base_concat + dequantize + base attention + vectorized joint
    correction) on `slices` (sequence, kv head) slices; extrapolate to the
    whole batch.

    With the GPU's output and diag rows, also check them against the
    oracle on the same slices (outside the timed region): selections equal
    up to epsilon ties of the normalised scores (1e-4 relative), and the
    output within max-abs 2e-3 (or one fp16 ulp where larger) of the oracle
    recomputed under the GPU's selection where a tie was crossed."""
    import numpy as np
    from oracle import quant as Q
    from oracle.attention import base_attention, vectorized_joint_correction
    from oracle.check import compare_selection, forced_selection, oracle_candidates, output_errors
    grp = spec["Hq"] // spec["Hkv"]
    total = 0.0
    par = dict(slices=0, rows=0, sel_exact=0, sel_tie=0, sel_bad=0, max_abs=0.0, rel_l2=0.0, bar_ratio=0.0)
    for seq, kvh in slice_ids(spec, slices):
        oc = oracle_slice_from_device(cache, seq, kvh, spec)
        Qg = q_np[seq, kvh * grp:(kvh + 1) * grp]
        kw = dict(kind="both", k_corr_scale=0.1, score_normalize=True, kscore_live=True, k_mode="exact")
        d = {}
        t0 = time.perf_counter()
        pids = oc.all_page_ids(0, 0)
        if spec.get("kivi"):  # attention.py:997-1008: the fp16 side buffer, no dequantisation
            Kh, Vh, _ = oc.read_base_hat_concat(0, 0, pids)
            Kh, Vh = Kh.astype(np.float32), Vh.astype(np.float32)
        else:
            Kc, Ks, Vc, Vs, _ = oc.read_base_concat(0, 0, pids)
            Kh = Q.dequantize(Kc, Ks, 32).astype(np.float32)
            Vh = Q.dequantize(Vc, Vs, 32).astype(np.float32)
        S, A, O = base_attention(Kh, Vh, Qg.astype(np.float32))
        dlt = vectorized_joint_correction(oc, 0, 0, pids, Qg, S, A, Vh, O, diag=d, **kw)
        ref = (O + dlt).astype(np.float16)
        total += time.perf_counter() - t0
        par["slices"] += 1
        if out_np is None or diag_np is None:
            continue
        Kcand, Vcand = oracle_candidates(oc, 0, 0, len(pids))
        rows = diag_np[seq, kvh * grp:(kvh + 1) * grp]
        ex, tie, bad = compare_selection(rows, d, Kcand, Vcand, eps=1e-4)
        par["rows"] += ex + tie + bad
        par["sel_exact"] += ex
        par["sel_tie"] += tie
        par["sel_bad"] += bad
        if tie:  # the oracle's output under the GPU's selection
            dlt = vectorized_joint_correction(oc, 0, 0, pids, Qg, S, A, Vh, O,
                                              force_sel=forced_selection(rows, Kcand, Vcand), **kw)
            ref = (O + dlt).astype(np.float16)
        mx, rel, ratio = output_errors(out_np[seq, kvh * grp:(kvh + 1) * grp], ref)
        par["max_abs"] = max(par["max_abs"], mx)
        par["rel_l2"] = max(par["rel_l2"], rel)
        par["bar_ratio"] = max(par["bar_ratio"], ratio)
    per_slice = total / max(par["slices"], 1)
    if out_np is not None:
        par["pass"] = bool(par["slices"] > 0 and par["sel_bad"] == 0 and par["bar_ratio"] <= 1.0
                           and par["rel_l2"] <= 1e-2)
        par["bar"] = ("selections equal up to epsilon ties (1e-4 relative); out within max-abs 2e-3 "
                      "(or 1 fp16 ulp) and rel-L2 1e-2 of the oracle under the GPU's selection")
        for k in ("max_abs", "rel_l2", "bar_ratio"):
            par[k] = float(f"{par[k]:.3g}")
    return per_slice * spec["B"] * spec["Hkv"] * 1e6, per_slice, par


def store_algorithmic_bytes(cache, cfg, B, H, T):
    """Bytes the prompt store must move, once each: the fp16 K and V rows
    read, the packed codes, int8 scale codes and fp16 masters, the page
    metadata (valid, has_meta, slot tables, fp16 error norms and sketches,
    fp32 sum of V_hat^2) and the 4-bit slots the call stored (with their
    fp16 scales) written.  The staging round trip of the slot payloads is
    not counted."""
    D, P = cfg.head_dim, -(-T // 16)
    ng, nvb, sd = D // 32, 4, cfg.sketch_dim
    pages = B * H * P
    rb = D * cfg.base_bits // 8
    slots = cache.next_slot.sum(0).tolist()  # stored K and V slots over the call's sequences
    terms = {"kv_fp16_in": 2 * B * H * T * D * 2,
             "codes": pages * 2 * 16 * rb,
             "scale_codes": pages * 2 * 16 * ng,
             "masters": pages * 2 * 2,
             "metadata": pages * (4 + 1 + 4 * (ng + nvb) + 2 * (ng + nvb) + 2 * ng * sd + 4),
             "slots": int(slots[0]) * (16 * 32 // 2 + 2) + int(slots[1]) * (4 * D // 2 + 2)}
    return int(sum(terms.values())), terms


def prefill_bench(args):
    """Config 4: causal prefill attention over dequantised K/V (layer.py:935-972)
    at B=4, 40 heads, D=128, T=8192, plus the quantize + pack + residual store
    of the same K/V into pages (timed separately).  One step = one layer's
    prefill attention for the batch."""
    os.environ.update(PAPER_ENV)
    import numpy as np
    import torch
    import care_kv
    c = PREFILL_CONFIG
    B, H, D, T = c["B"], c["H"], c["D"], c["T"]
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    g = torch.Generator(device=dev).manual_seed(c["seed"])
    q = torch.randn(B, H, T, D, generator=g, device=dev).half()
    # K, V ~ N(0,1) with per-channel log-normal scales (sigma 1)
    kx = (torch.randn(B, H, T, D, generator=g, device=dev) *
          torch.exp(torch.randn(B, H, 1, D, generator=g, device=dev))).half()
    vx = (torch.randn(B, H, T, D, generator=g, device=dev) *
          torch.exp(torch.randn(B, H, 1, D, generator=g, device=dev))).half()
    # store path: quantize + pack + residual candidates/slots into the paged cache
    P = math.ceil(T / 16)
    cfg = care_kv.CacheConfig(num_layers=1, num_heads=H, num_kv_heads=H, head_dim=D, page_size=16,
                              max_pages=P + 4, base_bits=c["bits"], group_size=32, k_channel_group=32,
                              v_token_block=4, sketch_dim=32, packed_base=True, scale_quant="int8",
                              store_budget_mode="ratio", store_budget_ratio=0.03, read_budget_ratio=0.0)
    cache = care_kv.CAREKVCache(cfg, device=dev, n_seq=B)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    cache.write_prefill(0, kx, vx, seqs=list(range(B)))  # warm-up (allocations, library load)
    torch.cuda.synchronize()
    # the store kernels (pass, slot scan, scatter), timed with HIP events on their stream around
    # their launches inside write_prefill, over fresh caches; and write_prefill's wall time
    store_us, store_ms_all = [], []
    for _ in range(5):
        cache = care_kv.CAREKVCache(cfg, device=dev, n_seq=B)
        k0, k1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        cache.store_events = (k0, k1)
        torch.cuda.synchronize()
        e0.record()
        cache.write_prefill(0, kx, vx, seqs=list(range(B)))  # the whole batch in one call, as CAREKVLayer.prefill
        e1.record()
        e1.synchronize()
        store_us.append(k0.elapsed_time(k1) * 1e3)
        store_ms_all.append(e0.elapsed_time(e1))
    store_kernels_us = float(np.median(store_us))
    store_ms = float(np.median(store_ms_all))
    store_bytes_alg, store_terms = store_algorithmic_bytes(cache, cfg, B, H, T)
    # K_hat, V_hat of the prefill path (fp16 group scales)
    kh = care_kv.quant_dequant(kx, c["bits"])
    vh = care_kv.quant_dequant(vx, c["bits"])
    del kx, vx
    out = torch.empty_like(q)
    for _ in range(args.warmup):
        care_kv.prefill_attention(q, kh, vh, out=out)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for _ in range(args.steps):
        care_kv.prefill_attention(q, kh, vh, out=out)
    ev1.record(stream)
    ev1.synchronize()
    ms = ev0.elapsed_time(ev1) / args.steps
    flops = 4.0 * B * H * D * (T * (T + 1) / 2)  # QK^T and PV over the causal triangle
    tflops = flops / (ms * 1e-3) / 1e12
    cpu = parity = None
    if not args.no_cpu_baseline:
        # the oracle (numpy restatement of _causal_attention_pure) on 512 query rows of two (sequence, head)
        # pairs, timed, extrapolated per row to the whole batch (the oracle's cost per row is one full
        # T-long score row, masked), and the GPU output of those rows checked against it
        import numpy as np
        from oracle.attention import causal_attention_pure
        rows = np.linspace(0, T - 1, 512).astype(np.int64)
        pairs = [(0, 0), (B - 1, H - 1)]
        t_cpu, mx_all, rel_all, ratio_all = 0.0, 0.0, 0.0, 0.0
        for (bb, hh) in pairs:
            qn = q[bb, hh:hh + 1].cpu().numpy()
            kn, vn = kh[bb, hh:hh + 1].cpu().numpy(), vh[bb, hh:hh + 1].cpu().numpy()
            t0 = time.perf_counter()
            ref, _ = causal_attention_pure(qn, kn, vn, causal=True, rows=rows)
            t_cpu += time.perf_counter() - t0
            got = out[bb, hh, torch.from_numpy(rows).to(dev)].cpu().numpy().astype(np.float32)
            # the bar of tests/test_gpu_prefill.py: max(2e-3, one fp16 ulp of the reference plus the
            # weight-rounding allowance 2^-11 sum_t a_t |v_t| from the fp64 softmax weights)
            s = (qn[0].astype(np.float64)[rows] @ kn[0].astype(np.float64).T) / math.sqrt(D)
            s = np.where(np.arange(T)[None, :] > rows[:, None], -np.inf, s)
            a = np.exp(s - s.max(-1, keepdims=True))
            allow = 2.0 ** -11 * (a / a.sum(-1, keepdims=True)) @ np.abs(vn[0].astype(np.float64))
            r32 = ref[0].astype(np.float32)
            bound = np.maximum(2e-3, np.spacing(np.abs(ref[0].astype(np.float16))).astype(np.float64) + allow)
            err = np.abs(got.astype(np.float64) - r32)
            mx = float(err.max())
            ratio = float((err / bound).max())
            rel = float(np.linalg.norm(got - r32) / max(np.linalg.norm(r32), 1e-30))
            mx_all, rel_all, ratio_all = max(mx_all, mx), max(rel_all, rel), max(ratio_all, ratio)
        per_row = t_cpu / (len(pairs) * len(rows))
        cpu_ms = per_row * B * H * T * 1e3
        try:
            import threadpoolctl
            cores = max([i.get("num_threads", 1) for i in threadpoolctl.threadpool_info()] + [1])
        except Exception:
            cores = int(os.environ.get("OMP_NUM_THREADS", "1"))
        cpu = {"value": round(cpu_ms, 1), "unit": "ms/step", "cores": cores, "kind": "port",
               "sample": f"{len(rows)} query rows of {len(pairs)} of {B * H} (sequence, head) pairs, numpy "
                         f"oracle ({per_row * 1e3:.3f} ms per row), extrapolated per row to {B * H * T} rows"}
        parity = {"rows": len(pairs) * len(rows), "max_abs": round(mx_all, 6), "rel_l2": round(rel_all, 6),
                  "bar_ratio": round(ratio_all, 3), "pass": bool(ratio_all <= 1.0 and rel_all <= 1e-2),
                  "bar": "out within max(2e-3, 1 fp16 ulp + 2^-11 sum_t a_t |v_t|) and rel-L2 1e-2 of the oracle"}
        log(f"[bench] c4 cpu oracle {per_row * 1e3:.3f} ms/row -> {cpu_ms / 1e3:.1f} s/step extrapolated; "
            f"parity {parity}")
    store_gbs = store_bytes_alg / (store_kernels_us * 1e-6) / 1e9
    tr = load_traffic("store", "c4")  # the three store kernels' counter traffic per call
    store_traffic = None if tr is None else tr.get("hbm_bytes_per_launch")
    log(f"[bench] c4 prefill attention {ms * 1e3:.1f} us/step, {flops / 1e12:.3f} TFLOP -> {tflops:.1f} TFLOP/s "
        f"({tflops / 2500 * 100:.1f}% of 2.5 PF fp16 dense); store kernels {store_kernels_us:.1f} us "
        f"({store_bytes_alg / 1e6:.1f} MB -> {store_gbs:.0f} GB/s, {store_gbs / 8000 * 100:.1f}% of 8 TB/s), "
        f"write_prefill {store_ms:.2f} ms wall for {B} sequences")
    line = {
        "metric": "CARE-KV prefill attention over dequantised K/V, TFLOP/s (Llama-2-13B shape, 8K prompt)",
        "value": round(tflops, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp16 MFMA (fp32 accumulate, fp32 softmax)", "data": "synthetic",
        "config": {"workload": c["workload"], "global_batch": B, "seq_len": T, "parallelism": "single-gpu",
                   "base": f"uniform INT{c['bits']} g=32 (K_hat/V_hat with fp16 group scales)", "causal": True},
        "roofline": {"bound": "mfma", "kernel": f"prefill_attn_kernel<{D}>", "achieved": round(tflops, 2),
                     "peak": 2500.0, "unit": "TFLOP/s", "frac": round(tflops / 2500.0, 4), "traffic": None,
                     "algorithmic_flops_per_launch": flops, "launch_us": round(ms * 1e3, 2)},
        "store": {"kernels": "store_pages_kernel + store_scan_kernel + store_slots_kernel",
                  "roofline": {"bound": "hbm", "achieved": round(store_gbs, 1), "peak": 8000.0, "unit": "GB/s",
                               "frac": round(store_gbs / 8000.0, 4), "traffic": store_traffic,
                               "algorithmic_bytes_per_call": store_bytes_alg, "terms": store_terms,
                               "launch_us": round(store_kernels_us, 2)},
                  "write_prefill_ms_wall": round(store_ms, 3)},
        "cpu_baseline": cpu,
        "parity": parity,
    }
    print(json.dumps(line), flush=True)
    if parity is not None and not parity["pass"]:
        log("[bench] PARITY FAILED: the GPU prefill attention differs from the oracle beyond the bar")
        sys.exit(3)


# prefill-time carekv_stored correction (layer.py:780-838) at the TinyLlama
# head shape with a 2048-token prompt; `--config pfc`
PFC_CONFIG = dict(Hq=32, Hkv=4, D=64, T=2048, rk=32, rv=32, seed=5,
                  workload="carekv_stored prefill correction, TinyLlama heads 32q/4kv D=64, 2048-token prompt")


def prefill_correction_bench(args):
    """One layer's carekv_stored prefill for one 2048-token prompt: the
    page store, the causal base attention with its LSE, and the sparse
    correction of every prompt row (carekv_prefill_correct), the last timed
    as the step.  CPU baseline: the oracle's prefill_stored on a bounded
    prefix of the prompt's rows, scaled by the causal work."""
    os.environ.update(PAPER_ENV)
    import numpy as np
    import torch
    import care_kv
    c = PFC_CONFIG
    Hq, Hkv, D, T = c["Hq"], c["Hkv"], c["D"], c["T"]
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    g = torch.Generator(device=dev).manual_seed(c["seed"])
    K = torch.randn(Hkv, T, D, generator=g, device=dev)
    for h in range(Hkv):
        K[h][:, torch.randperm(D, generator=g, device=dev)[:4]] *= 8.0
    K = K.half()
    V = torch.randn(Hkv, T, D, generator=g, device=dev).half()
    q = torch.randn(T, Hq, D, generator=g, device=dev).half()
    cfg = care_kv.CacheConfig(num_layers=1, num_heads=Hq, num_kv_heads=Hkv, head_dim=D, page_size=16,
                              max_pages=T // 16 + 4, base_bits=3, group_size=32, k_channel_group=32,
                              v_token_block=4, sketch_dim=32, packed_base=True, scale_quant="int8",
                              store_budget_mode="ratio", store_budget_ratio=0.03, read_budget_ratio=0.0,
                              read_budget_mode="absolute", read_abs_k=c["rk"], read_abs_v=c["rv"],
                              route_policy="joint")
    cache = care_kv.CAREKVCache(cfg, device=dev, n_seq=1)
    cache.write_prefill(0, K, V)
    kh, vh = care_kv.quant_dequant(K, 3), care_kv.quant_dequant(V, 3)
    ob, lse = care_kv.prefill_attention(q.transpose(0, 1), kh, vh, return_lse=True)
    for _ in range(args.warmup):
        out = care_kv.prefill_correction(cache, 0, q, kh, vh, lse[0] if lse.dim() == 3 else lse)
    torch.cuda.synchronize()
    lse2 = lse[0] if lse.dim() == 3 else lse
    stream = torch.cuda.current_stream(dev)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for _ in range(args.steps):
        out = care_kv.prefill_correction(cache, 0, q, kh, vh, lse2)
    ev1.record(stream)
    ev1.synchronize()
    ms = ev0.elapsed_time(ev1) / args.steps
    ev0.record(stream)
    for _ in range(args.steps):
        care_kv.prefill_attention(q.transpose(0, 1), kh, vh, return_lse=True)
    ev1.record(stream)
    ev1.synchronize()
    base_ms = ev0.elapsed_time(ev1) / args.steps
    rows_s = T / (ms * 1e-3)
    # the causal QK^T and PV the correction pass recomputes per row (the
    # streaming pass re-derives the base weights from the LSE)
    flops = 4.0 * Hq * D * (T * (T + 1) / 2)
    tflops = flops / (ms * 1e-3) / 1e12
    log(f"[bench] pfc: correction {ms * 1e3:.1f} us for {T} rows ({rows_s:.0f} rows/s, {tflops:.1f} TFLOP/s "
        f"causal-equivalent); base attention + LSE {base_ms * 1e3:.1f} us")
    cpu = None
    if not args.no_cpu_baseline:
        from oracle.attention import prefill_stored
        from oracle.cache import OCache, OCfg
        from oracle.store import write_pages_for_kv_head
        n = 256  # a prefix of the prompt: the oracle's per-row work grows with the row
        oc = OCache(OCfg(num_layers=1, num_heads=Hq, num_kv_heads=Hkv, head_dim=D, page_size=16,
                         max_pages=n // 16 + 4, base_bits=3, group_size=32, k_channel_group=32, v_token_block=4,
                         sketch_dim=32, read_budget_mode="absolute", read_abs_k=c["rk"], read_abs_v=c["rv"],
                         route_policy="joint", store_budget_mode="ratio", store_budget_ratio=0.03))
        Kn, Vn, Qn = K[:, :n].cpu().numpy(), V[:, :n].cpu().numpy(), q[:n].cpu().numpy()
        hats = [write_pages_for_kv_head(oc, 0, h, Kn[h], Vn[h]) for h in range(Hkv)]
        okh, ovh = np.stack([a for a, _ in hats]), np.stack([b for _, b in hats])
        t0 = time.perf_counter()
        prefill_stored(oc, 0, Qn.transpose(1, 0, 2), okh, ovh, k_mode="exact", kind="both", k_corr_scale=0.1,
                       score_normalize=True, kscore_live=True)
        sec = time.perf_counter() - t0
        scale = (T * (T + 1)) / (n * (n + 1))  # causal work ratio
        cpu = {"value": round(sec * scale * 1e6, 1), "unit": "us/step", "cores": 1, "kind": "port",
               "sample": f"oracle prefill_stored over the first {n} prompt rows ({sec:.2f} s), scaled by the "
                         f"causal work ratio x{scale:.0f}"}
        log(f"[bench] cpu oracle {sec:.2f} s for {n} rows -> {sec * scale:.1f} s extrapolated")
    line = {
        "metric": "CARE-KV carekv_stored prefill correction us per layer-prompt (TinyLlama heads, 2K prompt)",
        "value": round(ms * 1e3, 2), "unit": "us/step", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp16 K_hat/V_hat, fp16 weights, fp32 scores", "data": "synthetic",
        "config": {"workload": c["workload"], "global_batch": 1, "seq_len": T, "parallelism": "single-gpu",
                   "base": "uniform INT3 g=32, int8 page scales", "store": "ratio 0.03 (1K+1V slot/page)",
                   "read": f"joint top-{c['rk'] + c['rv']} per row, KSCORE_LIVE, normalize, exact"},
        "rows_per_s": round(rows_s, 1), "base_attention_us": round(base_ms * 1e3, 2),
        "roofline": {"bound": "mfma", "kernel": "decode_stream_kernel<64,16,0,true> (+ select, apply)",
                     "achieved": round(tflops, 3), "peak": 2500.0, "unit": "TFLOP/s",
                     "frac": round(tflops / 2500.0, 5), "traffic": None, "algorithmic_flops_per_launch": flops,
                     "launch_us": round(ms * 1e3, 2)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


# carekv_eval prefill correction (layer.py:792-806, the in-memory residuals)
# at the TinyLlama head shape with a 2048-token prompt; `--config pev`
PEV_CONFIG = dict(Hq=32, Hkv=4, D=64, T=2048, ratio=0.05, seed=7, n_cpu=512,
                  workload="carekv_eval prefill correction, TinyLlama heads 32q/4kv D=64, 2048-token prompt, "
                           "ratio 0.05")


def prefill_eval_bench(args):
    """One layer's carekv_eval prefill for one 2048-token prompt: the
    correction of every row from the full residuals K - K_hat, V - V_hat
    (carekv_prefill_eval) over the causal base attention of K_hat / V_hat,
    timed as the step.  Every (row t, query head) re-reads its t + 1 tokens'
    K, K_hat, V, V_hat rows and takes four D-long products per token (q.K_hat,
    q.r_K, |r_V|^2, |V_hat - o|^2): the roofline prices those 8 D flops per
    (head, row, token) against the fp32 peak.  CPU baseline: the oracle's
    prefill_eval on a prefix of the rows (the causal rows before n depend on
    nothing after n), scaled by the causal work; the same prefix of the GPU
    output is compared with it under the GPU's base output."""
    import numpy as np
    import torch
    import care_kv
    c = PEV_CONFIG
    Hq, Hkv, D, T = c["Hq"], c["Hkv"], c["D"], c["T"]
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    g = torch.Generator(device=dev).manual_seed(c["seed"])
    K = torch.randn(Hkv, T, D, generator=g, device=dev).half()
    V = torch.randn(Hkv, T, D, generator=g, device=dev).half()
    q = torch.randn(Hq, T, D, generator=g, device=dev).half()
    kh, vh = care_kv.quant_dequant(K, 3), care_kv.quant_dequant(V, 3)
    ob = care_kv.prefill_attention(q, kh, vh)
    ob = ob[0] if ob.dim() == 4 else ob
    for _ in range(args.warmup):
        out = care_kv.prefill_eval(q, K, V, kh, vh, ob, ratio=c["ratio"])
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for _ in range(args.steps):
        out = care_kv.prefill_eval(q, K, V, kh, vh, ob, ratio=c["ratio"])
    ev1.record(stream)
    ev1.synchronize()
    ms = ev0.elapsed_time(ev1) / args.steps
    flops = 8.0 * D * Hq * (T * (T + 1) / 2)
    tflops = flops / (ms * 1e-3) / 1e12
    log(f"[bench] pev: carekv_eval correction {ms * 1e3:.1f} us for {T} rows x {Hq} heads "
        f"({tflops:.2f} TFLOP/s of the 8 D flops per (head, row, token))")
    cpu, parity = None, None
    if not args.no_cpu_baseline:
        from oracle.attention import prefill_eval as oracle_prefill_eval
        n = c["n_cpu"]
        qn, Kn, Vn = q[:, :n].cpu().numpy(), K[:, :n].cpu().numpy(), V[:, :n].cpu().numpy()
        khn, vhn, obn = kh[:, :n].cpu().numpy(), vh[:, :n].cpu().numpy(), ob[:, :n].cpu().numpy()
        t0 = time.perf_counter()
        ref = oracle_prefill_eval(qn, Kn, Vn, khn, vhn, ratio=c["ratio"], o_base=obn)  # (n, Hq, D)
        sec = time.perf_counter() - t0
        scale = (T * (T + 1)) / (n * (n + 1))
        cpu = {"value": round(sec * scale * 1e6, 1), "unit": "us/step", "cores": 1, "kind": "port",
               "sample": f"oracle prefill_eval over the first {n} prompt rows of all {Hq} heads ({sec:.2f} s), "
                         f"scaled by the causal work ratio x{scale:.1f}"}
        got = out[:, :n].float().cpu().numpy().transpose(1, 0, 2)
        ref = np.asarray(ref, dtype=np.float32)
        err = np.abs(got - ref)
        rel = float(np.linalg.norm(got - ref) / max(float(np.linalg.norm(ref)), 1e-30))
        parity = {"rows": n, "heads": Hq, "max_abs": float(err.max()), "rel_l2": rel,
                  "rows_within_2e-3": float((err.reshape(n, Hq, D).max(-1) <= 2e-3).mean()),
                  "pass": bool(rel <= 1e-2),
                  "bar": "rel-L2 1e-2 of the oracle over the prefix (rows whose selection meets a near-tie may "
                         "differ by a corrected token; the GPU tests bound those)"}
        log(f"[bench] cpu oracle {sec:.2f} s for {n} rows -> {sec * scale:.1f} s extrapolated; parity {parity}")
    line = {
        "metric": "CARE-KV carekv_eval prefill correction us per layer-prompt (TinyLlama heads, 2K prompt)",
        "value": round(ms * 1e3, 2), "unit": "us/step", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp16 inputs, fp32 scores and products", "data": "synthetic",
        "config": {"workload": c["workload"], "global_batch": 1, "seq_len": T, "parallelism": "single-gpu",
                   "base": "uniform INT3 g=32 quant-dequant (K_hat, V_hat)", "kind": "both, output_aware V score"},
        "roofline": {"bound": "mfma", "kernel": "prefill_eval_kernel<64>", "achieved": round(tflops, 3),
                     "peak": 157.3, "unit": "TFLOP/s", "frac": round(tflops / 157.3, 4), "traffic": None,
                     "algorithmic_flops_per_launch": flops, "launch_us": round(ms * 1e3, 2),
                     "note": "fp32 arithmetic against the fp32 peak"},
        "cpu_baseline": cpu,
        "parity": parity,
    }
    print(json.dumps(line), flush=True)
    if parity is not None and not parity["pass"]:
        sys.exit(3)


# end-to-end random-init TinyLlama-1.1B through
# patch_llama_model, paper-best configuration; `--config c5`
E2E_CONFIG = dict(B=32, T=2048, new=256, seed=5,
                  workload="config5 TinyLlama-1.1B random init, 22 layers, B=32, prompt 2048, 256 greedy tokens")


def e2e_bench(args):
    """Greedy generation through the patched HF model: carekv_stored prefill
    (store + prefill attention + stored-slot correction) and one CARE-KV
    decode step per layer and token, paper-best knobs (README.md:151-165).
    value = generated tokens / s over the whole generate call.  Quality:
    teacher-forced top-1 agreement of the unpatched fp16 model with the
    generated tokens (the reference model cannot run on the GPU box)."""
    os.environ.update(PAPER_ENV)
    os.environ.update(CAREKV_PREFILL_MODE="carekv_stored", CAREKV_CORRECTION_IMPL="vectorized")
    import torch
    from transformers import LlamaConfig, LlamaForCausalLM
    import care_kv
    c = E2E_CONFIG
    B, T, new = c["B"], c["T"], c["new"]
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    mc = LlamaConfig(hidden_size=2048, intermediate_size=5632, num_hidden_layers=22, num_attention_heads=32,
                     num_key_value_heads=4, vocab_size=32000, max_position_embeddings=4096, rms_norm_eps=1e-5,
                     initializer_range=0.02)
    mc._attn_implementation = "eager"
    torch.manual_seed(c["seed"])
    t0 = time.time()
    with dev:  # initialise on the device
        model = LlamaForCausalLM(mc).half().eval()
        ref = LlamaForCausalLM(mc).half().eval()
    ref.load_state_dict(model.state_dict())
    log(f"[bench] c5: models built in {time.time() - t0:.1f}s")
    P = (T + new) // 16 + 4
    cc = care_kv.CacheConfig(num_layers=22, num_heads=32, num_kv_heads=4, head_dim=64, page_size=16, max_pages=P,
                             base_bits=3, group_size=32, k_channel_group=32, v_token_block=4, sketch_dim=32,
                             packed_base=True, scale_quant="int8", store_budget_mode="absolute", store_abs_k=2,
                             store_abs_v=4, read_budget_mode="absolute", read_abs_k=2, read_abs_v=2,
                             route_policy="joint", read_budget_ratio=0.0, correction_impl="vectorized")
    care_kv.patch_llama_model(model, cc)
    g = torch.Generator().manual_seed(c["seed"] + 1)
    ids = torch.randint(0, 32000, (B, T), generator=g).to(dev)
    with torch.no_grad():
        model.generate(ids[:, :64], max_new_tokens=4, do_sample=False, use_cache=True)  # warm-up
        care_kv.reset_all_caches(model)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        out = model.generate(ids, max_new_tokens=new, do_sample=False, use_cache=True)
        torch.cuda.synchronize()
        sec = time.perf_counter() - t0
        care_kv.reset_all_caches(model)
        # time the prefill alone (one forward over the prompt, the cache written)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        model(ids, use_cache=False)
        torch.cuda.synchronize()
        pre = time.perf_counter() - t1
        care_kv.reset_all_caches(model)
        # teacher-forced agreement: fp16 eager attention on the generated sequence
        agree = 0
        for b0 in range(0, B, 4):
            lg = ref(out[b0:b0 + 4, :-1], use_cache=False).logits[:, T - 1:]
            agree += int((lg.argmax(-1) == out[b0:b0 + 4, T:]).sum())
            del lg
    agreement = agree / (B * new)
    tps = B * new / sec
    log(f"[bench] c5: generate {sec:.2f} s for {B}x{new} tokens ({tps:.0f} tokens/s), prefill alone {pre * 1e3:.0f} ms; "
        f"teacher-forced top-1 agreement with fp16 attention {agreement:.4f}")
    line = {
        "metric": "CARE-KV end-to-end greedy generation tokens/s (TinyLlama-1.1B shape, random init, INT3 comb+ex)",
        "value": round(tps, 1), "unit": "tokens/s", "n_gpus": 1, "steps": 1, "warmup": 1,
        "ms_per_step": round(sec * 1e3, 1), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp16 model, int3-packed KV", "data": "synthetic (random-init weights, random token ids)",
        "config": {"workload": c["workload"], "global_batch": B, "seq_len": T, "new_tokens": new,
                   "parallelism": "single-gpu",
                   "carekv": "carekv_stored prefill, store abs 2K/4V, read abs 2K/2V joint, KSCORE_LIVE, exact"},
        "prefill_ms": round(pre * 1e3, 1),
        "top1_agreement_vs_fp16_attention": round(agreement, 4),
        "roofline": None, "cpu_baseline": None,
    }
    print(json.dumps(line), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="c3", choices=sorted(CONFIGS) + ["c4", "c5", "pfc", "pev"])
    ap.add_argument("--cpu-slices", type=int, default=16)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--eager", action="store_true",
                    help="time eager launches of the decode step instead of replays of its HIP graph")
    ap.add_argument("--split-pages", type=int, default=None)
    ap.add_argument("--no-correction", action="store_true",
                    help="time the base attention path only (streaming pass + split combine)")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="instead of the decode, time a plain device copy of this many MiB (counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}): the decode path is embarrassingly "
              "parallel over (sequence, kv head) and is not built for several GPUs in this tree.", file=sys.stderr)
        sys.exit(2)
    if args.copy_mib > 0:
        copy_calibration(args.copy_mib, args.steps)
        return
    if args.config == "c4":
        prefill_bench(args)
        return
    if args.config == "pfc":
        prefill_correction_bench(args)
        return
    if args.config == "pev":
        prefill_eval_bench(args)
        return
    if args.config == "c5":
        e2e_bench(args)
        return
    os.environ.update(PAPER_ENV)
    import numpy as np
    import torch
    import care_kv
    spec = CONFIGS[args.config]
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    B, Hq, Hkv, D, N = spec["B"], spec["Hq"], spec["Hkv"], spec["D"], spec["N"]
    P = math.ceil(N / 16)
    kivi = spec.get("kivi")
    base_kw = dict(base_bits=kivi, base_quantizer="kivi_style") if kivi else dict(base_bits=3)
    if spec.get("packed"):
        base_kw.update(kivi_packed=True, kivi_tail_pages=4)
    cfg = care_kv.CacheConfig(num_layers=1, num_heads=Hq, num_kv_heads=Hkv, head_dim=D, page_size=16,
                              max_pages=P + 4, group_size=32, k_channel_group=32, v_token_block=4,
                              sketch_dim=32, packed_base=True, scale_quant="int8", store_budget_mode="ratio",
                              store_budget_ratio=0.03, read_budget_ratio=0.0, read_budget_mode="absolute",
                              read_abs_k=spec["rk"], read_abs_v=spec["rv"], route_policy="joint", **base_kw)
    t0 = time.time()
    cache = care_kv.CAREKVCache(cfg, device=dev, n_seq=B)
    for b in range(B):
        K, V = gen_kv(torch, spec, b, dev)
        cache.write_prefill(0, K, V, seqs=[b])
        del K, V
    torch.cuda.synchronize()
    log(f"[bench] {args.config}: cache built in {time.time() - t0:.1f}s "
        f"({torch.cuda.memory_allocated() / 2**30:.2f} GiB allocated)")
    gq = torch.Generator(device=dev).manual_seed(spec["seed"] + 7)
    q = torch.randn(B, Hq, D, generator=gq, device=dev).half()
    out, diag = care_kv.decode_attention(cache, 0, q, diag_cap=512, split_pages=args.split_pages)
    torch.cuda.synchronize()
    diag_np = diag.cpu().numpy()
    out_first = out.clone()
    stream_bytes, nbytes, k_slots, v_union = algorithmic_bytes(spec, cfg, cache, diag_np)
    corr = not args.no_correction
    for _ in range(args.warmup):
        care_kv.decode_attention(cache, 0, q, out=out, split_pages=args.split_pages, correction=corr)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    # per-step phase events (recorded once so that the handles exist), re-recorded by the library on the
    # launch stream around its kernels
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(5)] for _ in range(args.steps)]
    for row in evs:
        for e in row:
            e.record(stream)
    torch.cuda.synchronize()
    # one decode step captured as a HIP graph (its four kernels; the caller's
    # q, output and workspace buffers), checked against eager launches on
    # replays with eager steps in between
    graph = None
    if not args.eager:
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(stream)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            care_kv.decode_attention(cache, 0, q, out=out, split_pages=args.split_pages, correction=corr)
            torch.cuda.synchronize()
            with torch.cuda.graph(graph, stream=side):
                care_kv.decode_attention(cache, 0, q, out=out, split_pages=args.split_pages, correction=corr)
        torch.cuda.synchronize()
        ref = torch.empty_like(out)
        for _ in range(3):
            care_kv.decode_attention(cache, 0, q, out=ref, split_pages=args.split_pages, correction=corr)
            out.zero_()
            graph.replay()
            torch.cuda.synchronize()
            if not torch.equal(out, ref):
                log("[bench] graph replay differs from the eager step")
                sys.exit(3)

    def timed(replay):
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        ev0.record(stream)
        for k in range(args.steps):
            if replay:
                graph.replay()
            else:
                care_kv.decode_attention(cache, 0, q, out=out, split_pages=args.split_pages, correction=corr)
        ev1.record(stream)
        ev1.synchronize()
        return ev0.elapsed_time(ev1) / args.steps

    # timed region: K steps with nothing else on the stream (graph replays
    # unless --eager), and the same K steps launched eagerly for reference;
    # the two modes alternate twice and the second round of each counts, so
    # that neither runs on a colder clock
    if graph is None:
        timed(False)
        ms_eager = ms_step = timed(False)
    else:
        timed(True)
        timed(False)
        ms_step = timed(True)
        ms_eager = timed(False)
    us_step = ms_step * 1e3
    # a second pass of K steps with per-kernel events for the phase split
    for k in range(args.steps):
        care_kv.decode_attention(cache, 0, q, out=out, split_pages=args.split_pages, correction=corr,
                                 phase_events=evs[k])
    torch.cuda.synchronize()
    phase = [sum(row[i].elapsed_time(row[i + 1]) for row in evs) / args.steps * 1e3 for i in range(4)]
    names = ["stream", "select", "apply", "combine"]
    gbps = nbytes / (ms_step * 1e-3) / 1e9
    stream_gbps = stream_bytes / (phase[0] * 1e-6) / 1e9
    log(f"[bench] {us_step:.1f} us/step ({'eager' if graph is None else 'graph replay'}; eager launches "
        f"{ms_eager * 1e3:.1f}), {nbytes / 1e9:.3f} GB algorithmic/step, {gbps:.0f} GB/s, "
        f"K slots {k_slots}, V union {v_union}")
    log("[bench] phases (us): " + ", ".join(f"{n} {t:.1f}" for n, t in zip(names, phase)) +
        f"; streaming kernel {stream_bytes / 1e9:.3f} GB -> {stream_gbps:.0f} GB/s")
    # the timed steps recompute the same output: it must not change
    deterministic = bool(torch.equal(out, out_first)) if corr else None
    cpu = None
    parity = None
    if not args.no_cpu_baseline:
        q_np = q.cpu().numpy()
        cpu_us, per_slice, parity = cpu_baseline(cache, spec, q_np, args.cpu_slices,
                                                 out_np=out_first.cpu().numpy() if corr else None,
                                                 diag_np=diag_np)
        if corr:
            parity["deterministic"] = deterministic
            parity["pass"] = bool(parity["pass"] and deterministic)
            log(f"[bench] parity vs oracle on {parity['slices']} slices: {parity}")
        try:
            import threadpoolctl
            info = threadpoolctl.threadpool_info()
            cores = max([i.get("num_threads", 1) for i in info] + [1])
        except Exception:
            cores = int(os.environ.get("OMP_NUM_THREADS", "1"))
        cpu = {"value": round(cpu_us, 1), "unit": "us/step", "cores": cores, "kind": "port",
               "sample": f"{len(slice_ids(spec, args.cpu_slices))} of {B * Hkv} (sequence, kv-head) slices of the same cache "
                         f"({per_slice:.3f} s each, numpy oracle), extrapolated x{B * Hkv}"}
        log(f"[bench] cpu oracle {per_slice:.3f} s/slice -> {cpu_us / 1e3:.1f} ms/step extrapolated")
    # the library runs the 4-query-head streaming kernel when a kv head has at
    # most 4 query heads and the split is a multiple of 16 pages
    sp = args.split_pages or care_kv.attention.default_split_pages(P, B * Hkv)
    packed = bool(spec.get("packed"))
    stream_kernel = ("decode_stream4_kernel" if Hq // Hkv <= 4 and sp % 16 == 0 and (packed or not kivi)
                     else "decode_stream_kernel")
    kbits, ksm = (2, 0) if packed else ((16, 0) if kivi else (cfg.base_bits, 1))
    tr = load_traffic(stream_kernel, args.config + ("_base" if args.no_correction else ""))
    traffic = None if tr is None else tr.get("hbm_bytes_per_launch")
    line = {
        "metric": "CARE-KV decode-attn us/step + HBM GB/s (% roofline), Mistral-7B shape 32K ctx",
        "value": round(us_step, 2), "unit": "us/step", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": ("int2-packed KIVI KV (per-channel K, per-token V scales)" if packed else
                  "fp16 K_hat/V_hat side buffer (KIVI INT2 values)" if kivi else "int3-packed KV") +
                 ", fp16 q/out, fp32 softmax", "data": "synthetic",
        "config": {"workload": spec["workload"], "global_batch": B, "seq_len": N, "parallelism": "single-gpu",
                   "base": (f"KIVI-style INT{kivi} (per-channel K, per-token V), packed pages" if packed else
                            f"KIVI-style INT{kivi} (per-channel K, per-token V), fp16 side buffer" if kivi
                            else "uniform INT3 g=32, int8 page scales"),
                   "store": "ratio 0.03 (1K+1V slot/page)",
                   "read": f"joint top-{spec['rk'] + spec['rv']} (K {spec['rk']} + V {spec['rv']}), "
                           "KSCORE_LIVE, normalize, exact"},
        "hbm_gbps": round(gbps, 1),
        "launch": "eager" if graph is None else "hip graph of one step, replayed",
        "us_per_step_eager": round(ms_eager * 1e3, 2),
        "phases_us": {n: round(t, 2) for n, t in zip(names, phase)},
        "roofline": {"bound": "hbm", "kernel": f"{stream_kernel}<{D},{kbits},{ksm}>",
                     "achieved": round(stream_gbps, 1), "peak": 8000.0, "unit": "GB/s",
                     "frac": round(stream_gbps / 8000.0, 4), "traffic": traffic,
                     "algorithmic_bytes_per_launch": int(stream_bytes), "launch_us": round(phase[0], 2),
                     "step_frac": round(gbps / 8000.0, 4), "step_algorithmic_bytes": int(nbytes)},
        "cpu_baseline": cpu,
        "parity": parity,
    }
    print(json.dumps(line), flush=True)
    if parity is not None and corr and not parity["pass"]:
        log("[bench] PARITY FAILED: the GPU output or selections differ from the oracle beyond the bar")
        sys.exit(3)


if __name__ == "__main__":
    main()
