"""Benchmark of WhiteMatter's attention hot path on one MI355X.

Headline (the "C2" configuration the baseline metric is quoted on): bf16 strict_causal_attention in
Jacobi mode, Q/K/V (8, 16, 2048, 128) ~ N(0,1)/sqrt(D), use_dummy_token=False,
packed documents per row with geometric lengths (mean 512, clipped to
[16, 2048], filled to exactly T), metadata from prepare_strict_causal_metadata,
forward + backward of sum(output). One step = one forward and one backward
of the attention operator on resident inputs; the metadata is prepared once
outside the timed region (the reference builds it once per model forward).

value = 14 * D * Hq * P / step time, P = visible (query, key) pairs counted
exactly from the metadata (the reference's FLOP convention,
benchmarks/_flop_counter.py:33-34). Per-kernel averages come from HIP events
on the launch stream; the dominant kernel gives the roofline object.
Secondary fields: C4 KV-pool decode GB/s, the C2 step with the dummy slot (the model's
call), C4 prefill forward TFLOP/s, C3 cyclic fwd+bwd
TFLOP/s (stride 4; strides 2 and 8 and the dummy-slot variant in `cyclic_variants`),
the fused KV-pool store GB/s beside the reference's eager steps, and the
packed-document schedule builder's latency beside the torch sequence,
the captured decode loop's per-token time beside eager launches, and the C5
harness (a 24-layer model's cyclic prefill and greedy decoding on these kernels).
The CPU baseline times the oracle (float32, dense mask) on a bounded sample.
"""

from __future__ import annotations

import argparse
import gc
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBPS = 8000.0  # MI355X HBM3E
CALIBRATION_BYTES = 256 << 20
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "c2_strict_jacobi_traffic.md")
KERNEL_NAMES = {  # rocprof kernel name prefix -> bench kernel key
    "wmx::attn_fwd_kernel": "attn_fwd",
    "wmx::bwd_delta_kernel": "bwd_delta",
    "wmx::attn_bwd_dq_kernel": "bwd_dq",
    "wmx::attn_bwd_dq_ds_kernel": "bwd_dq",
    "wmx::attn_bwd_dkv_kernel": "bwd_dkv",
    "wmx::decode_split_kernel<128, 1>": "decode_split_g1",  # C4 decode, 16 KV heads
    "wmx::decode_split_kernel<128, 2>": "decode_split_g2",  # C4 decode, 8 KV heads
    "wmx::decode_split_kernel": "decode_split",
    "wmx::decode_combine_kernel": "decode_combine",
    "wmx::kv_premix_kernel": "kv_premix",
    "wmx::kv_mix_kernel": "kv_mix",
    "wmx::kv_router_kernel": "kv_router",
    "wmx::kv_router_reduce_kernel": "kv_router_reduce",
}
METRIC = "attn fwd+bwd TFLOP/s (bf16, T=2048) and % MFMA peak; decode GB/s"


def geometric_documents(batch: int, length: int, seed: int, mean: int = 512, lo: int = 16, hi: int = 2048):
    """Per-row document ids: lengths ~ Geometric(1/mean) clipped to [lo, hi],
    appended until the row holds `length` tokens; the last is truncated to
    fill exactly, and a remainder below `lo` is merged into the previous one."""
    rng = np.random.default_rng(seed)
    rows = []
    for _ in range(batch):
        sizes = []
        while sum(sizes) < length:
            sizes.append(int(np.clip(rng.geometric(1.0 / mean), lo, hi)))
        sizes[-1] -= sum(sizes) - length
        if sizes[-1] < lo and len(sizes) > 1:
            sizes[-2] += sizes.pop()
        rows.append(np.repeat(np.arange(len(sizes)), sizes))
    return torch.from_numpy(np.stack(rows)).long()


def visible_pairs(metadata) -> int:
    """Visible (query, key) pairs of a varlen schedule: segment s with nq queries
    and nk keys is bottom-right causal, so query i sees nk - nq + i + 1 keys."""
    total = 0
    for qs, qe, ks, ke in metadata.segments:
        nq, nk = qe - qs, ke - ks
        total += nq * (nk - nq) + nq * (nq + 1) // 2
    return total


class Timer:
    """HIP-event timing on the current stream."""

    def __init__(self):
        self.start = torch.cuda.Event(enable_timing=True)
        self.stop = torch.cuda.Event(enable_timing=True)

    def __call__(self, fn, reps: int) -> float:
        torch.cuda.synchronize()
        issue = time.perf_counter()
        self.start.record()
        for _ in range(reps):
            fn()
        self.stop.record()
        # host time to issue the steps: below the GPU time the GPU never waits for the host
        self.host_ms = (time.perf_counter() - issue) * 1e3 / reps
        torch.cuda.synchronize()
        return self.start.elapsed_time(self.stop) / reps


def strict_jacobi_setup(device, seed=0, batch=8, heads=16, length=2048, dim=128):
    from white_matter_amd import prepare_strict_causal_metadata

    gen = torch.Generator().manual_seed(seed)
    scale = dim**-0.5
    q, k, v = (
        (torch.randn(batch, heads, length, dim, generator=gen) * scale).to(device, torch.bfloat16)
        for _ in range(3)
    )
    docs = geometric_documents(batch, length, seed).to(device)
    t0 = time.perf_counter()
    metadata = prepare_strict_causal_metadata(docs, length)
    meta_ms = (time.perf_counter() - t0) * 1e3
    return q, k, v, docs, metadata, meta_ms


def kernel_times(q, k, v, metadata, reps):
    """Average duration (ms) of each kernel of one forward+backward, launched
    through the C ABI between its own pair of HIP events on the current
    stream, `reps` rounds of the four kernels in step order (dK/dV stores the
    dS that dQ reads), averaged over the later half of the rounds. The
    launches are queued without waiting for them; the returned function reads
    the events after the caller has synchronised."""
    from white_matter_amd import _kernels, _native
    from white_matter_amd.strict_causal_attention import _covering_schedule, _keys_unique_code, _schedule_flags, _work_units

    batch, heads, length, dim = q.shape
    metadata = _covering_schedule(metadata, batch, length, k.shape[2])  # the schedule the operator runs
    max_q, max_k, flags = _schedule_flags(metadata)
    varlen = _kernels.Varlen(
        metadata.query_indices, metadata.key_indices, metadata.cu_queries, metadata.cu_keys,
        metadata.cu_queries.numel() - 1, max_q, max_k, length, k.shape[2], _keys_unique_code(flags), flags & 15,
        *_work_units(metadata, query_extent=length),
    )
    vis = _kernels.Visibility(varlen=varlen)
    out = torch.zeros(batch, length, heads, dim, device=q.device, dtype=torch.bfloat16)
    o = out.transpose(1, 2)
    lse = torch.empty(batch, heads, length, device=q.device, dtype=torch.float32)
    dout = torch.ones_like(o)
    dq, dk, dv = (torch.zeros_like(t) for t in (q, k, v))
    delta = torch.empty_like(lse)
    args = _kernels._base_args(q, k, v, o, lse, dim**-0.5, vis, length)
    args.dout, args.delta = dout.data_ptr(), delta.data_ptr()
    args.do_stride = _kernels._strides(dout)
    args.dq, args.dk, args.dv = dq.data_ptr(), dk.data_ptr(), dv.data_ptr()
    args.dq_stride, args.dk_stride, args.dv_stride = (_kernels._strides(t) for t in (dq, dk, dv))
    need = _native.attn_bwd_workspace_size(args)
    workspace = torch.empty(max(need, 16), device=q.device, dtype=torch.uint8)
    args.workspace, args.workspace_bytes = workspace.data_ptr(), need
    dev = q.device
    calls = {
        "attn_fwd": lambda: _native.attn_fwd(args, dev),
        "bwd_delta": lambda: _native.attn_bwd_preprocess(args, dev),
        "bwd_dkv": lambda: _native.attn_bwd_dkv(args, dev),
        "bwd_dq": lambda: _native.attn_bwd_dq(args, dev),
    }
    for fn in calls.values():
        fn()
    # the kernels in step order, each launch between its own pair of events
    events = {name: [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
              for name in calls}
    torch.cuda.synchronize()
    for i in range(reps):
        for name, fn in calls.items():
            begin, end = events[name][i]
            begin.record()
            fn()
            end.record()
    keep = (workspace, out, dout, dq, dk, dv, delta, lse, varlen)

    def result() -> dict[str, float]:
        # read once the launches have run (the caller synchronises): the
        # average of the later half, the GPU's clock settling over the first
        # ~25 ms of back-to-back work after an idle period
        assert keep
        later = reps // 2
        return {name: sum(b.elapsed_time(e) for b, e in pairs[later:]) / (reps - later) for name, pairs in events.items()}

    return result


def decode_setup(device, seed=1, batch=32, heads=16, kv_heads=16, dim=128, capacity=8192):
    gen = torch.Generator().manual_seed(seed)
    q = (torch.randn(batch, heads, 1, dim, generator=gen) * dim**-0.5).to(device, torch.bfloat16)
    k = torch.empty(batch, kv_heads, capacity, dim, device=device, dtype=torch.bfloat16).normal_(0, dim**-0.5)
    v = torch.empty_like(k).normal_(0, dim**-0.5)
    lengths = torch.from_numpy(np.random.default_rng(seed).integers(512, 8192, size=batch, endpoint=True)).to(device)
    return q, k, v, lengths


def cpu_baseline(q, k, v, metadata, budget_s: float):
    """The oracle (float32 dense-mask softmax, forward + backward) on single rows
    of the C2 batch, on this host's CPU threads, until `budget_s` has passed."""
    from oracle import attention as ref

    threads = torch.get_num_threads()
    batch, heads, length, dim = q.shape
    qi = metadata.query_indices.cpu().numpy()
    cq = metadata.cu_queries.cpu().numpy()
    keep_all = None
    done_pairs, elapsed, rows = 0, 0.0, 0
    meta_np = {
        "query_indices": qi,
        "key_indices": metadata.key_indices.cpu().numpy(),
        "cu_queries": cq,
        "cu_keys": metadata.cu_keys.cpu().numpy(),
        "key_extent": metadata.key_extent,
    }
    keep_all = ref.schedule_keep(meta_np, batch, length, k.shape[2])
    while elapsed < budget_s:
        b = rows % batch  # cycle over the batch rows until the budget is spent
        qb, kb, vb = (t[b : b + 1].float().cpu().requires_grad_() for t in (q, k, v))
        keep = keep_all[b : b + 1, None]
        t0 = time.perf_counter()
        out = ref.masked_attention(qb, kb, vb, keep, dim**-0.5, dtype=torch.float32)
        out.sum().backward()
        elapsed += time.perf_counter() - t0
        done_pairs += int(keep.sum())
        rows += 1
    flops = 14 * dim * heads * done_pairs
    return {
        "value": flops / elapsed / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{rows} single-row passes over the {batch} rows of the C2 batch (all {heads} heads, "
        f"T={length}), fp32 forward + backward, {elapsed:.1f} s; visible-pair FLOPs as the GPU value",
    }


def algorithmic_bytes(q, k, v, pairs) -> dict[str, int]:
    """HBM bytes each kernel must move at least once per launch: its operands
    read and its results written (bf16 tensors, fp32 LSE and delta, bf16 dS
    for the visible pairs of every query head, which the dK/dV kernel writes
    and the dQ kernel reads)."""
    t = q.numel() * 2  # Q, O, dO, dQ each
    kv = k.numel() * 2 + v.numel() * 2
    rows = q.shape[0] * q.shape[1] * q.shape[2] * 4  # LSE or delta
    ds = 2 * q.shape[1] * pairs
    return {
        "attn_fwd": 2 * t + kv + rows,  # Q, K, V in; O, LSE out
        "bwd_delta": 2 * t + rows,  # O, dO in; delta out
        "bwd_dq": t + k.numel() * 2 + ds,  # K, dS in; dQ out
        "bwd_dkv": 2 * t + 2 * kv + 2 * rows + ds,  # Q, dO, K, V, LSE, delta in; dK, dV, dS out
    }


def binding_roof(flops: int, nbytes: int) -> float:
    """The roof (TFLOP/s) that binds a kernel of this arithmetic intensity:
    min(MFMA peak, AI x HBM peak); the ridge is 2.5 PFLOP/s / 8 TB/s = 312.5
    FLOP/byte."""
    return min(PEAK_BF16_TFLOPS, flops / nbytes * PEAK_HBM_GBPS / 1e3) if nbytes else PEAK_BF16_TFLOPS


def kernel_roofline(flops: int, nbytes: int, ms: float) -> dict:
    """The roofline object of one kernel against the roof its arithmetic
    intensity (algorithmic FLOPs over algorithmic bytes) makes binding: HBM
    bytes per second below the ridge, MFMA FLOPs per second above it; the MFMA
    fraction is reported beside it either way."""
    ai = flops / nbytes if nbytes else float("inf")
    tflops = flops / (ms * 1e-3) / 1e12
    gbps = nbytes / (ms * 1e-3) / 1e9
    hbm_bound = ai * PEAK_HBM_GBPS / 1e3 < PEAK_BF16_TFLOPS
    achieved, peak = (gbps, PEAK_HBM_GBPS) if hbm_bound else (tflops, PEAK_BF16_TFLOPS)
    return {
        "bound": "hbm" if hbm_bound else "mfma",
        "achieved": round(achieved, 2),
        "peak": peak,
        "unit": "GB/s" if hbm_bound else "TFLOP/s",
        "frac": round(achieved / peak, 4),
        "ai_flop_per_byte": round(ai, 1),
        "mfma_tflops": round(tflops, 2),
        "mfma_frac": round(tflops / PEAK_BF16_TFLOPS, 4),
    }


def step_floors(q, k, v, pairs, hbm, flops) -> dict:
    """Byte floors of one fwd+bwd step at 8 TB/s and the MFMA fraction each
    caps the step at: the chosen kernels' algorithmic bytes (with the bf16 dS
    round trip between dK/dV and dQ), and the algorithm's own (Q, K, V, O, dO,
    LSE read once; O, dQ, dK, dV written once)."""
    design = sum(hbm.values())
    t = q.numel() * 2
    kv = k.numel() * 2 + v.numel() * 2
    rows = q.shape[0] * q.shape[1] * q.shape[2] * 4
    own = (t + kv + t + t + rows) + (t + t + kv)
    out = {}
    for name, nbytes in (("design", design), ("algorithm", own)):
        ms = nbytes / (PEAK_HBM_GBPS * 1e9) * 1e3
        out[name] = {"bytes": nbytes, "ms": round(ms, 4), "mfma_cap_frac": round(flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)}
    return out


def measured_traffic(kernel: str) -> int | None:
    """HBM bytes per launch of `kernel` (FETCH_SIZE + WRITE_SIZE scaled by the
    calibration copy) from the JSON block of the committed rocprof summary of
    this workload, or None when there is none."""
    try:
        with open(TRAFFIC_PROFILE) as f:
            text = f.read()
        block = text.split("```json", 1)[1].split("```", 1)[0]
        entry = json.loads(block)["kernels"][kernel]
        return int(entry["fetch_bytes"] + entry["write_bytes"])
    except (OSError, IndexError, KeyError, ValueError):
        return None


def pmc_summary(dirs) -> dict:
    """Per-kernel averages of FETCH_SIZE and WRITE_SIZE (KiB per dispatch,
    summed over counter dimensions) from rocprofv3 --pmc --output-format csv
    directories, converted to bytes with the factor the same counters read on
    the calibration copy (torch.neg over CALIBRATION_BYTES in and out)."""
    import csv
    import glob

    per = {}  # (kernel, dispatch) -> counter -> value
    for d in dirs:
        for path in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            with open(path) as f:
                for row in csv.DictReader(f):
                    key = (row["Kernel_Name"], path, row["Dispatch_Id"])
                    counters = per.setdefault(key, {})
                    name = row["Counter_Name"]
                    counters[name] = counters.get(name, 0.0) + float(row["Counter_Value"])
    calib = {}
    sums = {}
    for (name, _, _), counters in per.items():
        for counter, value in counters.items():
            if "neg_kernel" in name:  # torch.neg's elementwise kernel: the calibration copy
                calib[counter] = max(calib.get(counter, 0.0), value)
            short = next((v for k, v in KERNEL_NAMES.items() if name.startswith(k) or name.startswith("void " + k)), None)
            if short:
                sums.setdefault(short, {}).setdefault(counter, []).append(value)
    out = {"calibration_bytes": CALIBRATION_BYTES, "calibration_counters_kib": calib, "kernels": {}}
    factor = {c: CALIBRATION_BYTES / v for c, v in calib.items() if v > 0}
    out["bytes_per_counter_unit"] = factor
    for short, counters in sums.items():
        entry = {}
        for counter, values in counters.items():
            avg = sum(values) / len(values)
            entry[counter.lower() + "_raw"] = avg
            if counter in factor:
                entry[{"FETCH_SIZE": "fetch_bytes", "WRITE_SIZE": "write_bytes"}.get(counter, counter)] = avg * factor[counter]
        out["kernels"][short] = entry
    return out


def main(argv=None) -> int:
    parser = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=100)
    parser.add_argument("--warmup", type=int, default=10)
    parser.add_argument("--kernel-reps", type=int, default=100)
    parser.add_argument("--cpu-budget", type=float, default=12.0, help="seconds of CPU baseline work")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-secondary", action="store_true", help="skip the secondary lines (decode, cyclic, store, builder, loops, C5)")
    parser.add_argument(
        "--only",
        choices=(
            "decode", "prefill", "cyclic", "kv_store", "kv_producer", "metadata", "decode_loop", "jacobi_dummy", "c5",
            "head_dim_96",
        ),
        help="print one secondary line as JSON and exit (for profiling that path alone)",
    )
    parser.add_argument(
        "--copy-calibration",
        action="store_true",
        help="first run one elementwise copy (torch.neg) of 256 MiB, the known-size kernel that scales FETCH_SIZE/WRITE_SIZE",
    )
    parser.add_argument(
        "--pmc-summary",
        nargs="+",
        metavar="DIR",
        help="summarise rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE output directories (no GPU work) and exit",
    )
    args = parser.parse_args(argv)
    if args.pmc_summary:
        print(json.dumps(pmc_summary(args.pmc_summary), indent=1))
        return 0
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2

    from white_matter_amd import strict_causal_attention

    device = torch.device("cuda:0")
    if args.copy_calibration:
        # one elementwise kernel that reads and writes exactly CALIBRATION_BYTES
        src = torch.ones(CALIBRATION_BYTES // 4, dtype=torch.float32, device=device)
        dst = torch.empty_like(src)
        torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst
    if args.only:
        lines = {
            "decode": decode_line,
            "prefill": prefill_line,
            "cyclic": cyclic_line,
            "kv_store": kv_store_line,
            "kv_producer": kv_producer_line,
            "metadata": metadata_line,
            "decode_loop": decode_loop_line,
            "jacobi_dummy": dummy_jacobi_line,
            "c5": c5_line,
            "head_dim_96": head_dim_96_line,
        }
        print(json.dumps({args.only: lines[args.only](device)}), flush=True)
        return 0
    q, k, v, docs, metadata, meta_ms = strict_jacobi_setup(device)
    batch, heads, length, dim = q.shape
    pairs = visible_pairs(metadata)
    dense_pairs = batch * length * (length - 1) // 2
    flops = 14 * dim * heads * pairs
    leaves = [t.clone().requires_grad_() for t in (q, k, v)]
    # the output gradient is an input of the backward, resident like Q/K/V
    grad_out = torch.ones(batch, length, heads, dim, device=device, dtype=torch.bfloat16)

    def step():
        out = strict_causal_attention(*leaves, metadata=metadata)
        torch.autograd.grad(out, leaves, grad_out)

    # The first call (which plans the schedule on the host) is timed apart,
    # as the reference's operator benchmark does. Then the per-kernel
    # durations are queued: their launches (kernel_reps rounds of the step's
    # four kernels, ~45 ms back to back) run while the host issues the warmup
    # steps, so the GPU goes from them into the timed steps without idling.
    # After an idle period of even a few milliseconds the GPU's clock takes
    # about 50 steps to settle (measured step times dip from 0.43 to 0.52 ms
    # around steps 6-10 after 0.5 s idle, and to 0.48 ms after a few ms).
    # A garbage collection first, so that none falls in the timed steps.
    gc.collect()
    torch.cuda.synchronize()
    first = time.perf_counter()
    step()
    torch.cuda.synchronize()
    first_ms = (time.perf_counter() - first) * 1e3
    read_kernels = kernel_times(q, k, v, metadata, args.kernel_reps)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    timer = Timer()
    ms = timer(step, args.steps)
    value = flops / (ms * 1e-3) / 1e12
    kernels = read_kernels()
    algorithmic = {  # FLOPs per launch credited to each kernel (10*D bwd = 8*D dkv + 2*D dq)
        "attn_fwd": 4 * dim * heads * pairs,
        "bwd_dq": 2 * dim * heads * pairs,
        "bwd_dkv": 8 * dim * heads * pairs,
        "bwd_delta": 0,
    }
    hbm = algorithmic_bytes(q, k, v, pairs)
    dominant = max(kernels, key=kernels.get)
    roofline = kernel_roofline(algorithmic[dominant], hbm[dominant], kernels[dominant])
    roofline.update(kernel=dominant, traffic=measured_traffic(dominant), algorithmic_bytes=hbm[dominant],
                    avg_ms=round(kernels[dominant], 4))
    floors = step_floors(q, k, v, pairs, hbm, flops)
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "host_ms_per_step": round(timer.host_ms, 4),
        "first_call_ms": round(first_ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "C2 strict_causal_attention Jacobi, packed geometric documents, fwd+bwd",
            "batch": batch,
            "heads": heads,
            "seq_len": length,
            "head_dim": dim,
            "documents": int(sum(int(docs[b].max()) + 1 for b in range(batch))),
            "visible_pairs": pairs,
            "dense_causal_pairs": dense_pairs,
            "dense_equivalent_tflops": round(14 * dim * heads * dense_pairs / (ms * 1e-3) / 1e12, 2),
            "metadata_ms": round(meta_ms, 3),
        },
        "roofline": roofline,
        "kernels": {
            name: {
                "avg_ms": round(t, 4),
                "algorithmic_tflops": round(algorithmic[name] / (t * 1e-3) / 1e12, 2),
                "frac_mfma": round(algorithmic[name] / (t * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                "algorithmic_gbps": round(hbm[name] / (t * 1e-3) / 1e9, 1),
                "frac_hbm": round(hbm[name] / (t * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4),
                "ai_flop_per_byte": round(algorithmic[name] / hbm[name], 1),
                "binding_roof_tflops": round(binding_roof(algorithmic[name], hbm[name]), 1),
                # below the ridge the HBM fraction is the fraction of the binding roof
                "frac_binding_roof": round(
                    min(hbm[name] / (t * 1e-3) / 1e9 / PEAK_HBM_GBPS, 1.0)
                    if binding_roof(algorithmic[name], hbm[name]) < PEAK_BF16_TFLOPS
                    else algorithmic[name] / (t * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
                    4,
                ),
            }
            for name, t in kernels.items()
        },
        "kernel_sum_ms": round(sum(kernels.values()), 4),
        "frac_of_peak_step": round(value / PEAK_BF16_TFLOPS, 4),
        "floors": floors,
    }

    if not args.no_secondary:
        line["decode"] = decode_line(device)
        line["jacobi_dummy"] = dummy_jacobi_line(device)
        line["head_dim_96"] = head_dim_96_line(device)
        line["prefill"] = prefill_line(device)
        line["cyclic"] = cyclic_line(device)
        line["cyclic_variants"] = [cyclic_line(device, 2), cyclic_line(device, 8), cyclic_line(device, 4, dummy=True)]
        line["kv_store"] = kv_store_line(device)
        line["kv_producer"] = kv_producer_line(device)
        line["metadata"] = metadata_line(device)
        line["decode_loop"] = decode_loop_line(device)
        line["c5"] = c5_line(device)

    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(q, k, v, metadata, args.cpu_budget)
    print(json.dumps(line), flush=True)
    return 0


def decode_line(device):
    """C4 decode: B=32, H=16, D=128, kv lengths ~ U{512..8192}, one token per
    row, over 16 KV heads (MHA, the primary line) and over 8 (GQA 2)."""
    from white_matter_amd import strict_causal_attention

    lines = {}
    for kv_heads in (16, 8):
        q, k, v, lengths = decode_setup(device, kv_heads=kv_heads)
        batch, _, capacity, dim = k.shape
        with torch.no_grad():
            fn = lambda: strict_causal_attention(q, k, v, query_start=lengths)  # noqa: E731
            for _ in range(3):
                fn()
            ms = Timer()(fn, 100)
        kv_bytes = int(lengths.sum()) * 2 * kv_heads * dim * 2
        other = q.numel() * 2 * 2 + batch * 8
        gbps = (kv_bytes + other) / (ms * 1e-3) / 1e9
        lines[kv_heads] = {
            "workload": f"C4 decode B=32 H=16 Hkv={kv_heads} D=128 kv_len~U[512,8192]",
            "ms": round(ms, 4),
            "gbps": round(gbps, 1),
            "frac_hbm": round(gbps / PEAK_HBM_GBPS, 4),
            "bytes": kv_bytes + other,
        }
    return {**lines[16], "kv_heads_8": lines[8]}


def dummy_jacobi_line(device, steps=30):
    """The C2 step as the model calls it with use_dummy_token (the k8 recipe):
    keys (8, 16, 2049, 128) with the dummy at slot 0, the same documents,
    forward + backward; FLOPs over the visible pairs (every query also sees
    the dummy)."""
    from white_matter_amd import prepare_strict_causal_metadata, strict_causal_attention

    q, k, v, docs, _, _ = strict_jacobi_setup(device)
    batch, heads, length, dim = q.shape
    gen = torch.Generator().manual_seed(4)
    k = torch.cat(((torch.randn(batch, heads, 1, dim, generator=gen) * dim**-0.5).to(device, k.dtype), k), 2)
    v = torch.cat(((torch.randn(batch, heads, 1, dim, generator=gen) * dim**-0.5).to(device, v.dtype), v), 2)
    metadata = prepare_strict_causal_metadata(docs, length, use_dummy_token=True)
    leaves = [t.clone().requires_grad_() for t in (q, k, v)]
    grad_out = torch.ones(batch, length, heads, dim, device=device, dtype=torch.bfloat16)

    def step():
        out = strict_causal_attention(*leaves, metadata=metadata, use_dummy_token=True)
        torch.autograd.grad(out, leaves, grad_out)

    for _ in range(3):
        step()
    ms = Timer()(step, steps)
    pairs = visible_pairs(metadata)
    tflops = 14 * dim * heads * pairs / (ms * 1e-3) / 1e12
    return {
        "workload": "C2 Jacobi with the dummy slot (use_dummy_token=True, keys 2049), fwd+bwd",
        "ms_per_step": round(ms, 4),
        "tflops": round(tflops, 2),
        "frac_mfma": round(tflops / PEAK_BF16_TFLOPS, 4),
    }


def head_dim_96_line(device, steps=30):
    """head_dim 96, the width of most of the reference's recipes: the C2 step
    (same documents and scaling) at D=96, and C4 decode at D=96 over 16 and 8
    KV heads; FLOPs and bytes counted as for the D=128 lines."""
    from white_matter_amd import strict_causal_attention

    q, k, v, docs, metadata, _ = strict_jacobi_setup(device, dim=96)
    batch, heads, length, dim = q.shape
    leaves = [t.clone().requires_grad_() for t in (q, k, v)]
    grad_out = torch.ones(batch, length, heads, dim, device=device, dtype=torch.bfloat16)

    def step():
        out = strict_causal_attention(*leaves, metadata=metadata)
        torch.autograd.grad(out, leaves, grad_out)

    for _ in range(3):
        step()
    ms = Timer()(step, steps)
    pairs = visible_pairs(metadata)
    tflops = 14 * dim * heads * pairs / (ms * 1e-3) / 1e12
    line = {
        "workload": "C2 Jacobi at head_dim 96 (8, 16, 2048, 96), packed geometric documents, fwd+bwd",
        "ms_per_step": round(ms, 4),
        "tflops": round(tflops, 2),
        "frac_mfma": round(tflops / PEAK_BF16_TFLOPS, 4),
    }
    del leaves, q, k, v, grad_out
    for kv_heads in (16, 8):
        q, k, v, lengths = decode_setup(device, kv_heads=kv_heads, dim=96)
        with torch.no_grad():
            fn = lambda: strict_causal_attention(q, k, v, query_start=lengths)  # noqa: E731
            for _ in range(3):
                fn()
            dms = Timer()(fn, 100)
        nbytes = int(lengths.sum()) * 2 * kv_heads * 96 * 2 + q.numel() * 2 * 2 + q.shape[0] * 8
        gbps = nbytes / (dms * 1e-3) / 1e9
        line[f"decode_kv_heads_{kv_heads}"] = {
            "workload": f"C4 decode B=32 H=16 Hkv={kv_heads} D=96 kv_len~U[512,8192]",
            "ms": round(dms, 4),
            "gbps": round(gbps, 1),
            "frac_hbm": round(gbps / PEAK_HBM_GBPS, 4),
        }
    return line


def cyclic_line(device, stride=4, dummy=False):
    """C3: cyclic fwd+bwd over a full pass of `stride` residue calls, packed
    documents from prepare_feedback_metadata. Without a dummy the bound is
    strict (strict_past=True); with one, key slot 0 is the dummy (id -1) and
    the bound is inclusive, as the model calls it."""
    from white_matter_amd import cyclic_attention, prepare_feedback_metadata

    batch, heads, length, dim = 8, 16, 2048, 128
    gen = torch.Generator().manual_seed(3)
    docs = geometric_documents(batch, length, 3).to(device)
    groups = [torch.arange(r, length, stride, device=device) for r in range(stride)]
    keys = length + int(dummy)
    metas = prepare_feedback_metadata(docs, groups, keys, use_dummy_token=dummy)
    k, v = ((torch.randn(batch, heads, keys, dim, generator=gen) * dim**-0.5).to(device, torch.bfloat16) for _ in range(2))
    qs = [(torch.randn(batch, heads, g.numel(), dim, generator=gen) * dim**-0.5).to(device, torch.bfloat16) for g in groups]
    kl, vl = k.clone().requires_grad_(), v.clone().requires_grad_()
    ql = [t.clone().requires_grad_() for t in qs]

    grads = [torch.ones(batch, heads, g.numel(), dim, device=device, dtype=torch.bfloat16) for g in groups]

    def full_pass():
        for r in range(stride):
            out = cyclic_attention(ql[r], kl, vl, query_stride=stride, query_offset=r, strict_past=not dummy,
                                   metadata=metas[r], backend="tilelang")
            torch.autograd.grad(out, (ql[r], kl, vl), grads[r])

    # a full collection now rather than inside the timed passes: among the
    # many tensors and schedules of a long run, one stalled the host for tens
    # of milliseconds while the GPU waited for the next launch (a stride-8
    # pass measured 11.7 instead of 1.38 ms)
    gc.collect()
    for _ in range(2):
        full_pass()
    ms = Timer()(full_pass, 10)
    # visible pairs of a full pass: per document, L(L-1)/2 strict pairs, or
    # L(L+1)/2 with the dummy (every query also sees slot 0)
    pairs = 0
    for b in range(batch):
        _, counts = torch.unique_consecutive(docs[b].cpu(), return_counts=True)
        pairs += int((counts * (counts + (1 if dummy else -1)) // 2).sum())
    tflops = 14 * dim * heads * pairs / (ms * 1e-3) / 1e12
    bound = "dummy slot, inclusive" if dummy else "strict_past"
    # byte floor of a pass under the per-call API: every residue call reads
    # all of K and V (forward, dK/dV, dQ) and writes full dK and dV; queries,
    # outputs and their gradients add up to one T-long set over the pass; the
    # bf16 dS of the visible pairs is written by dK/dV and read by dQ
    qset = batch * heads * length * dim * 2
    kv = k.numel() * 2
    rows = batch * heads * length * 4
    floor_bytes = (
        (qset + 2 * stride * kv + qset + rows)  # forward
        + (2 * qset + rows)  # delta
        + (2 * qset + 2 * stride * kv + 2 * rows + 2 * stride * kv)  # dK/dV (dS below)
        + (stride * kv + qset)  # dQ
        + 2 * 2 * heads * pairs  # dS written and read
    )
    floor_ms = floor_bytes / (PEAK_HBM_GBPS * 1e9) * 1e3
    return {
        "workload": f"C3 cyclic stride {stride} full pass, {bound}, geometric documents, fwd+bwd",
        "ms_per_pass": round(ms, 4),
        "tflops": round(tflops, 2),
        "frac_mfma": round(tflops / PEAK_BF16_TFLOPS, 4),
        "byte_floor_ms": round(floor_ms, 4),
        "frac_byte_floor": round(floor_ms / ms, 4),
    }


def prefill_line(device, seed=1, batch=32, heads=16, dim=128, chunk=256):
    """C4 prefill: a chunk of 256 new queries per row after a cached prefix
    P_b ~ U{512..8192} (query_start = P as a tensor, kv_lengths = P + 256),
    forward only, FLOPs 4*D*Hq*sum_b sum_i (P_b + i). The kernel's work is a
    fixed cycle count; under sustained load the power manager first lowers
    the GPU clock (about 2 ms into it) and then settles it, so 30 warm-up calls
    (about 12 ms) precede the 20 timed ones, which then see the settled clock
    a long prefill runs at rather than the transient."""
    from white_matter_amd import strict_causal_attention

    gen = torch.Generator().manual_seed(seed)
    prefix = torch.from_numpy(np.random.default_rng(seed).integers(512, 8192, size=batch, endpoint=True))
    capacity = int(prefix.max()) + chunk
    q = (torch.randn(batch, heads, chunk, dim, generator=gen) * dim**-0.5).to(device, torch.bfloat16)
    k = torch.empty(batch, heads, capacity, dim, device=device, dtype=torch.bfloat16).normal_(0, dim**-0.5)
    v = torch.empty_like(k).normal_(0, dim**-0.5)
    start, lengths = prefix.to(device), (prefix + chunk).to(device)
    with torch.no_grad():
        fn = lambda: strict_causal_attention(q, k, v, query_start=start, kv_lengths=lengths)  # noqa: E731
        for _ in range(30):
            fn()
        ms = Timer()(fn, 20)
    pairs = int(prefix.sum()) * chunk + batch * chunk * (chunk - 1) // 2
    tflops = 4 * dim * heads * pairs / (ms * 1e-3) / 1e12
    # Q read, O and LSE written, each row's K and V read up to its last visible slot
    nbytes = 2 * q.numel() * 2 + batch * heads * chunk * 4 + int(lengths.sum()) * heads * dim * 2 * 2
    roof = kernel_roofline(4 * dim * heads * pairs, nbytes, ms)
    return {
        "workload": f"C4 prefill B={batch} H=Hkv={heads} D={dim}, {chunk} new queries after a cached prefix ~U[512,8192], fwd",
        "ms": round(ms, 4),
        "tflops": round(tflops, 2),
        "frac_mfma": round(tflops / PEAK_BF16_TFLOPS, 4),
        "pairs": pairs,
        "algorithmic_bytes": nbytes,
        "roofline": roof,
        "byte_floor_ms": round(nbytes / (PEAK_HBM_GBPS * 1e9) * 1e3, 4),
    }


def decode_loop_line(device, batch=8, heads=16, kv_heads=8, channels=8, dim=64, layers=24, prefix=1024, tokens=128):
    """Cached decoding at the 24-layer model's shape: per token, 24 layers each
    attend from (B, 16, 1, 64) queries to one of 8 pool channels (B, 8, N, 64),
    then the token's keys/values are K-normed, rotated and stored, and the
    slot counter advances. 128 tokens after a 1024-token prefix, replayed from
    one DecodeLoop graph, beside the same launches issued eagerly. Bytes per
    token: every layer's K and V reads of its channel up to the current
    length, the queries, outputs and the store."""
    from white_matter_amd import DecodeLoop

    gen = torch.Generator().manual_seed(9)
    capacity = prefix + 1 + tokens
    folded = channels * kv_heads
    keys = torch.empty(batch, folded, capacity, dim, device=device, dtype=torch.bfloat16).normal_(0, 1)
    values = torch.empty_like(keys).normal_(0, 1)
    length = torch.tensor([prefix + 1], device=device)
    weight = torch.ones(channels, dim, device=device)
    angle = torch.arange(capacity, device=device)[:, None].float() * torch.logspace(0, -4, dim // 2, device=device)[None]
    angle = torch.cat((angle, angle), -1)
    loop = DecodeLoop(keys, values, length, [layer % channels for layer in range(layers)], weight, angle.cos(), angle.sin(),
                      query_heads=heads)
    loop.query.copy_(torch.randn(loop.query.shape, generator=gen).to(device, torch.bfloat16))
    loop.new_key.copy_(torch.randn(loop.new_key.shape, generator=gen).to(device, torch.bfloat16))
    loop.new_value.copy_(torch.randn(loop.new_value.shape, generator=gen).to(device, torch.bfloat16))
    start = length.clone()

    def run(fn):
        length.copy_(start)
        loop.seen = prefix + 1
        torch.cuda.synchronize()
        return Timer()(fn, tokens)

    with torch.inference_mode():
        graph_ms = run(loop)
        eager_ms = run(loop.step)
    lengths = sum(prefix + t for t in range(tokens)) / tokens  # keys seen per token (dummy included)
    per_token = layers * (2 * batch * kv_heads * lengths * dim * 2 + 2 * batch * heads * dim * 2)
    per_token += 4 * batch * folded * dim * 2
    return {
        "workload": f"decode loop: {layers} layers, Q ({batch},{heads},1,{dim}) over {channels} pool channels "
        f"({batch},{kv_heads},N,{dim}), {tokens} tokens after a {prefix}-token prefix, store included",
        "graph_ms_per_token": round(graph_ms, 4),
        "eager_ms_per_token": round(eager_ms, 4),
        "gbps": round(per_token / (graph_ms * 1e-3) / 1e9, 1),
        "frac_hbm": round(per_token / (graph_ms * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4),
        "bytes_per_token": int(per_token),
    }


def c5_line(device, batch=8, length=2048, tokens=128, seed=13):
    """C5 end to end: the 24-layer model (d 1024, 16x64 query heads, 8 KV heads,
    8 pool channels over 25 sources, vocab 151936, bf16, random weights) on 8
    rows of 2048 uniform random token ids packed into geometric documents
    (mean 512): the cyclic prefill (8 groups, 3 passes, metadata and packed
    schedules built in the call) through the HIP attention and store kernels,
    then 128 greedy decode steps replayed from one graph. hipBLASLt (torch)
    runs the projections, routers and MLPs."""
    from white_matter_amd.cyclic_pass import FeedbackConfig, FeedbackModel, GreedyDecoder, forward_cyclic

    config = FeedbackConfig()
    model = FeedbackModel(config, device=device, seed=seed)
    gen = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, config.vocab_size, (batch, length), generator=gen).to(device)
    docs = geometric_documents(batch, length, seed).to(device)
    capacity = length + 1 + tokens
    forward_cyclic(model, ids, docs, capacity=capacity)  # warm-up: GEMM heuristics, allocator
    timer = Timer()
    prefill_ms = timer(lambda: forward_cyclic(model, ids, docs, capacity=capacity), 2)
    hidden, keys, values, positions = forward_cyclic(model, ids, docs, capacity=capacity)
    decoder = GreedyDecoder.after_prefill(model, hidden, keys, values, positions, docs)
    decode_ms = timer(decoder, tokens)
    return {
        "workload": f"C5: {config.num_layers} layers, d {config.hidden_size}, {config.num_heads}x{config.head_dim} "
        f"query heads, {config.num_kv_heads} KV heads, {config.num_kv_channels} channels over {config.num_sources} "
        f"sources, vocab {config.vocab_size}; B={batch} T={length} geometric documents, {config.cyclic_groups} "
        f"groups x {config.num_passes} passes, then {tokens} greedy tokens from one graph",
        "prefill_ms": round(prefill_ms, 2),
        "prefill_tokens_per_s": round(batch * length / (prefill_ms * 1e-3)),
        "decode_ms_per_token": round(decode_ms, 4),
        "decode_tokens_per_s": round(batch / (decode_ms * 1e-3)),
        "data": "synthetic token ids, random-initialised weights",
    }


def metadata_line(device, batch=8, length=2048, reps=20):
    """Packed-document schedule for the C2 documents (8 rows of 2048 slots,
    geometric lengths): prepare_strict_causal_metadata as a caller sees it
    (returns with the host segment list), through the HIP builder, through the
    reference's torch sequence on the same GPU, and that sequence on the host
    CPU (the reference's CPU path)."""
    from white_matter_amd import prepare_feedback_metadata, prepare_strict_causal_metadata
    from white_matter_amd.strict_causal_attention import _torch_schedule

    docs = geometric_documents(batch, length, 0)
    on_gpu = docs.to(device)

    def wall(fn, n):
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / n

    hip_ms = wall(lambda: prepare_strict_causal_metadata(on_gpu, length), reps)
    torch_ms = wall(lambda: _torch_schedule(on_gpu, length, 0, None, False), reps)
    cpu_ms = wall(lambda: _torch_schedule(docs, length, 0, None, False), 5)
    # the model's per-forward cyclic metadata at the default stride 8, every residue
    stride = 8
    slots_cpu = [torch.arange(r, length, stride) for r in range(stride)]
    slots_gpu = [p.to(device) for p in slots_cpu]
    feedback_hip = wall(lambda: prepare_feedback_metadata(on_gpu, slots_gpu, length + 1), reps)
    feedback_cpu = wall(lambda: prepare_feedback_metadata(docs, slots_cpu, length + 1), 5)
    return {
        "workload": f"prepare_strict_causal_metadata, C2 documents B={batch} T={length}, host segment list included",
        "hip_ms": round(hip_ms, 4),
        "torch_on_gpu_ms": round(torch_ms, 4),
        "torch_on_cpu_ms": round(cpu_ms, 4),
        "cpu_threads": torch.get_num_threads(),
        "feedback": {
            "workload": f"prepare_feedback_metadata, same documents, stride {stride} (all residues), dummy slot",
            "hip_ms": round(feedback_hip, 4),
            "cpu_ms": round(feedback_cpu, 4),
        },
    }


def kv_store_line(device, batch=8, channels=8, heads=16, tokens=2048, dim=64, seed=5):
    """KV-pool store at the 24-layer model's pool shape (8 channels, 16 heads
    of 64): bf16 keys/values straight from the per-channel projection (the
    (C, B*T, H*D) product viewed as (B, C, H, T, D), no copy), fp32 RoPE
    tables, written into a (B, C, H, T+1, D) pool after the dummy slot. Bytes:
    keys and values read once and written once, cos/sin and the weights read
    once, the slots. The reference's eager steps (rms_norm, weight, RoPE,
    casts, two index_copy_) are timed beside it on the same GPU."""
    import torch.nn.functional as F

    from white_matter_amd import kv_pool

    gen = torch.Generator().manual_seed(seed)
    shape = (channels, batch, tokens, heads, dim)
    k_proj = torch.randn(*shape, generator=gen).to(device, torch.bfloat16)
    v_proj = torch.randn(*shape, generator=gen).to(device, torch.bfloat16)
    key, value = (t.permute(1, 0, 3, 2, 4) for t in (k_proj, v_proj))  # (B, C, H, T, D) views
    weight = (1 + 0.1 * torch.randn(channels, dim, generator=gen)).to(device)
    angle = torch.rand(batch, tokens, dim // 2, generator=gen).to(device) * 100
    cos, sin = torch.cat((angle, angle), -1).cos(), torch.cat((angle, angle), -1).sin()
    keys = torch.zeros(batch, channels, heads, tokens + 1, dim, device=device, dtype=torch.bfloat16)
    values = torch.zeros_like(keys)
    slots = torch.arange(1, tokens + 1, device=device)

    def fused():
        kv_pool.write_pool(key, value, weight, cos, sin, keys, values, slots)

    def eager():
        normed = F.rms_norm(key, (dim,), None, 1e-6) * weight.view(1, channels, 1, 1, dim).to(key.dtype)
        c, s = cos[:, None, None].to(key.dtype), sin[:, None, None].to(key.dtype)
        k = ((normed * c) + (torch.cat((-normed[..., dim // 2 :], normed[..., : dim // 2]), -1) * s)).to(value.dtype)
        keys.index_copy_(3, slots, k)
        values.index_copy_(3, slots, value)

    with torch.no_grad():
        for fn in (fused, eager):
            for _ in range(3):
                fn()
        ms = Timer()(fused, 50)
        eager_ms = Timer()(eager, 10)
    elements = batch * channels * heads * tokens * dim
    moved = elements * 2 * 4 + 2 * batch * tokens * dim * 4 + channels * dim * 4 + tokens * 8
    gbps = moved / (ms * 1e-3) / 1e9
    return {
        "workload": f"KV-pool store B={batch} C={channels} H={heads} T={tokens} D={dim}, bf16 projection views, fp32 RoPE",
        "ms": round(ms, 4),
        "gbps": round(gbps, 1),
        "frac_hbm": round(gbps / PEAK_HBM_GBPS, 4),
        "bytes": moved,
        "eager_reference_ms": round(eager_ms, 4),
    }


def kv_producer_line(device, batch=8, tokens=256, seed=9):
    """The KV-pool producer ahead of the per-channel projection for one group
    of the C5 pass (8 rows x 256 tokens, the block input and 24 layer outputs
    as 25 fp32 sources of 1024, 8 channels): the HIP kernels around the
    router GEMM (kv_pool.projection_inputs) against the same steps as torch
    operations on the same GPU (the harness's formulation of the reference's
    `_project`). Bytes of the HIP kernels: sources read once (fp32), both
    premixed stacks written (bf16), read again by the mixture, the channels
    written; the router GEMM reads the premixed stacks once more."""
    from white_matter_amd.cyclic_pass import FeedbackConfig, FeedbackModel, HipKernels

    config = FeedbackConfig()
    model = FeedbackModel(config, device=device, seed=seed)
    gen = torch.Generator(device=device).manual_seed(seed)
    for side in "kv":  # content weights in the routers, not only the prior
        weight, _ = model.router[side]
        weight.copy_((torch.randn(weight.shape, generator=gen, device=device) * 0.003).to(weight.dtype))
    sources, hidden, channels = config.num_sources, config.hidden_size, config.num_kv_channels
    read = len(model.router_read)  # sources the routers read (router_layer_stride)
    stacked = torch.randn(batch, tokens, sources, hidden, generator=gen, device=device)
    with torch.no_grad():
        for _ in range(3):
            HipKernels.mix(model, stacked)
            model.projection_inputs(stacked)
        ms = Timer()(lambda: HipKernels.mix(model, stacked), 20)
        eager_ms = Timer()(lambda: model.projection_inputs(stacked), 10)
    rows = batch * tokens
    premix = rows * sources * hidden * (4 + 2 * 2)
    mix = rows * (2 * sources * hidden * 2 + 2 * channels * sources * 2 + 2 * channels * hidden * 2)
    gemm = 2 * (rows * read * hidden * 2 + channels * sources * read * hidden * 2)
    moved = premix + mix + gemm
    return {
        "workload": f"KV-pool producer, one C5 group: B={batch} T={tokens}, {sources} fp32 sources x {hidden}, "
        f"{channels} channels (premix, router GEMM over {read} sources: router_layer_stride "
        f"{config.router_layer_stride}, routed sum, mix norm, gain)",
        "ms": round(ms, 4),
        "gbps": round(moved / (ms * 1e-3) / 1e9, 1),
        "frac_hbm": round(moved / (ms * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4),
        "bytes": {"premix": premix, "mix": mix, "router_gemm": gemm},
        "torch_ops_ms": round(eager_ms, 4),
    }


if __name__ == "__main__":
    sys.exit(main())
