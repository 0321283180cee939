"""Benchmark of the MI355X attention hot path.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
                    [--only decode|prefill] [--workload config3|config4]

Headline (the JSON `value`): paged decode attention at the Qwen3-8B shape —
batch 256, 32 query / 8 KV heads, head_dim 128, bf16, block 16, context
lengths uniform in [1024, 8192] (seed 0), a pool of 1.1x the needed blocks and
random-permutation block tables.  One step = one decode-attention call over
the whole batch (the split-KV partition kernel plus the LSE merge), inputs
resident in HBM.  value = algorithmic bytes per step / time per step (GB/s).

Also reported on the same line:
  roofline      the decode call against the 8 TB/s HBM peak, timed with HIP
                events on the launch stream;
  cpu_baseline  the oracle's restatement of the reference's PyTorch decode path
                (qwen3/paged_attention.py:39-122) on the host cores, over a
                bounded sample (the first 64 sequences) of the same workload;
  prefill       varlen causal prefill at the Qwen3-0.6B shape (8 sequences,
                lengths uniform in [64, 2048], 16/8 heads) in TFLOP/s against
                the 2.5 PFLOP/s bf16 dense MFMA peak, plus its slot write.
Prints exactly one JSON line on stdout (progress goes to stderr).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
METRIC = "paged-decode attn GB/s & %HBM peak; varlen prefill TFLOPS & %MFMA peak"


def log(msg: str) -> None:
    sys.stderr.write(f"[bench] {msg}\n")
    sys.stderr.flush()


def decode_inputs(lens, hq, hkv, dev, seed=0, slack=0.1, block_size=16, head_dim=128):
    import numpy as np
    import torch

    g = torch.Generator(device=dev).manual_seed(seed)
    pages = [(L + block_size - 1) // block_size for L in lens]
    nb = int(np.ceil(sum(pages) * (1 + slack)))
    perm = torch.randperm(nb, generator=g, device=dev).to(torch.int32)
    bt = torch.full((len(lens), max(pages)), -1, dtype=torch.int32, device=dev)
    off = 0
    for b, n in enumerate(pages):
        bt[b, :n] = perm[off:off + n]
        off += n
    k = torch.randn(nb, hkv, block_size, head_dim, generator=g, device=dev, dtype=torch.bfloat16)
    v = torch.randn(nb, hkv, block_size, head_dim, generator=g, device=dev, dtype=torch.bfloat16)
    q = torch.randn(len(lens), hq, head_dim, generator=g, device=dev, dtype=torch.bfloat16)
    sl = torch.tensor([L - 1 for L in lens], dtype=torch.int32, device=dev)
    rows = torch.arange(len(lens), dtype=torch.int32, device=dev)
    return dict(q=q, k=k, v=v, bt=bt, seq_lens=sl, row_ids=rows, pages=pages, nb=nb)


def decode_bytes(lens, hq, hkv, head_dim=128, block_size=16):
    """Algorithmic HBM bytes of one decode call: K and V of every attended
    token, q in, out, the block-table entries and per-row lengths/ids."""
    pages = sum((L + block_size - 1) // block_size for L in lens)
    B = len(lens)
    return (sum(lens) * hkv * head_dim * 2 * 2 + 2 * B * hq * head_dim * 2 + 4 * pages + 8 * B)


def time_steps(fn, steps, warmup):
    """W untimed warmups, then K timed steps bracketed by synchronize; each
    step is also bracketed by events on torch's current stream (where the
    kernels are launched).  Returns (wall ms/step, mean event ms/step)."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(steps)]
    t0 = time.perf_counter()
    for s, e in ev:
        s.record()
        fn()
        e.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    evt = sum(s.elapsed_time(e) for s, e in ev) / steps
    return wall, evt


def bench_decode(args, dev):
    import torch

    from oracle import inputs as oi
    from qwen3_engine_from_scratch_amd.kernels.paged_attention import (
        paged_attention_decode_hip, paged_decode_workspace_bytes)

    if args.workload == "config4":
        lens, wname = oi.config4_lengths(), ("long-context split-KV paged decode, Qwen3-8B shape: "
                                             "B=8, L~U[32768,131072]")
    else:
        lens, wname = oi.config3_lengths(), ("paged decode attention, Qwen3-8B shape: B=256, "
                                             "L~U[1024,8192]")
    hq, hkv = 32, 8
    log(f"decode inputs: B={len(lens)} sumL={sum(lens)}")
    t = decode_inputs(lens, hq, hkv, dev)
    out = torch.empty_like(t["q"])
    ws = torch.empty(paged_decode_workspace_bytes(len(lens), hq, 128, t["bt"].shape[1], 16),
                     dtype=torch.uint8, device=dev)

    def step():
        paged_attention_decode_hip(t["q"], t["k"], t["v"], t["bt"], t["seq_lens"], t["row_ids"],
                                   16, out=out, workspace=ws)

    wall_ms, evt_ms = time_steps(step, args.steps, args.warmup)
    nbytes = decode_bytes(lens, hq, hkv)
    log(f"decode: {evt_ms * 1e3:.1f} us/call (events), {wall_ms * 1e3:.1f} us/step (wall)")
    res = dict(lens=lens, wname=wname, bytes=nbytes, wall_ms=wall_ms, evt_ms=evt_ms, t=t)
    return res


def cpu_baseline_decode(res, n_seq=64):
    """The oracle (restated reference PyTorch decode path) on the host cores
    over the first n_seq sequences of the same workload (same bytes)."""
    import torch

    from oracle import decode as od

    t = res["t"]
    lens = res["lens"][:n_seq]
    pages = [(L + 15) // 16 for L in lens]
    bt = t["bt"][:n_seq].cpu()
    used = torch.cat([bt[b, :n].long() for b, n in enumerate(pages)])
    remap = torch.full((t["nb"],), -1, dtype=torch.long)
    remap[used] = torch.arange(used.numel())
    k_cpu = t["k"][used.to(t["k"].device)].cpu()
    v_cpu = t["v"][used.to(t["v"].device)].cpu()
    bt_small = torch.full_like(bt, -1)
    m = bt >= 0
    bt_small[m] = remap[bt[m].long()].to(torch.int32)
    q_cpu = t["q"][:n_seq].cpu()
    sl = t["seq_lens"][:n_seq].cpu()
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    log(f"cpu baseline: {n_seq} sequences, {sum(pages)} pages, {torch.get_num_threads()} threads")
    t0 = time.perf_counter()
    od.paged_attention_ref(q_cpu, k_cpu, v_cpu, bt_small, sl, None, 16)
    dt = time.perf_counter() - t0
    nbytes = decode_bytes(lens, 32, 8)
    return {"value": round(nbytes / dt / 1e9, 4), "unit": "GB/s",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"first {n_seq} of {len(res['lens'])} sequences ({sum(lens)} tokens, "
                      f"{sum(pages)} pages), one pass of the oracle's per-page loop, "
                      f"{dt:.2f} s"}


PROFILE_DIR = Path(__file__).resolve().parent / "profiles"
TRAFFIC_PROFILE = "paged_decode_stream_b256_qwen3_8b.md"


def profiled_traffic(name: str):
    """HBM bytes per launch measured offline with rocprofv3 --pmc FETCH_SIZE /
    WRITE_SIZE (scaled by a known-size copy) and recorded in profiles/<name>."""
    f = PROFILE_DIR / name
    if not f.exists():
        return None
    for line in f.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(float(line.split(":", 1)[1]))
    return None


def bench_prefill(args, dev):
    import torch

    from oracle import inputs as oi
    from qwen3_engine_from_scratch_amd import _lib
    from qwen3_engine_from_scratch_amd.kernels.flash_attention_varlen import flash_attention_prefill

    if args.prefill_workload == "steady":
        # 8 x 4096 tokens, non-causal: every query tile sweeps every key tile,
        # no masking and no ragged tail (the kernel's steady-state rate).
        lens = [4096] * 8
        g = torch.Generator(device=dev).manual_seed(0)
        q = torch.randn(sum(lens), 16, 128, device=dev, generator=g).to(torch.bfloat16)
        k = torch.randn(sum(lens), 8, 128, device=dev, generator=g).to(torch.bfloat16)
        v = torch.randn(sum(lens), 8, 128, device=dev, generator=g).to(torch.bfloat16)
        cu = torch.tensor([0] + [4096 * (i + 1) for i in range(8)], dtype=torch.int32, device=dev)
        out = torch.empty_like(q)

        def sstep():
            flash_attention_prefill(q, k, v, cu, 128 ** -0.5, 16, 8, 128, max_seqlen=4096,
                                    causal=False, out=out)

        _, s_evt = time_steps(sstep, args.steps, args.warmup)
        flops = 4 * 128 * 16 * sum(L * L for L in lens)
        tflops = flops / (s_evt * 1e-3) / 1e12
        log(f"prefill (steady, 8x4096 non-causal): {s_evt * 1e3:.1f} us/call, {tflops:.1f} TFLOP/s")
        return {"workload": "varlen non-causal prefill, 8 x 4096 tokens, 16/8 heads, head_dim 128, bf16",
                "value": round(tflops, 2), "unit": "TFLOP/s", "ms_per_step": round(s_evt, 5),
                "flops": flops,
                "roofline": {"bound": "mfma", "achieved": round(tflops, 2),
                             "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                             "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": None}}

    c = oi.config2_prefill()
    q, k, v = c.q.to(dev), c.k.to(dev), c.v.to(dev)
    cu = c.cu_seqlens.to(dev)
    out = torch.empty_like(q)
    mx = max(c.lens)

    def step():
        flash_attention_prefill(q, k, v, cu, c.scale, 16, 8, 128, max_seqlen=mx, out=out)

    wall_ms, evt_ms = time_steps(step, args.steps, args.warmup)
    flops = 2 * 128 * 16 * sum(L * (L + 1) for L in c.lens)
    tflops = flops / (evt_ms * 1e-3) / 1e12
    log(f"prefill: {evt_ms * 1e3:.1f} us/call, {tflops:.1f} TFLOP/s")

    # slot write of the same prefill into a block-16 pool (one launch)
    kb = torch.zeros(c.num_blocks, 1, 8, 16, 128, dtype=torch.bfloat16, device=dev)
    vb = torch.zeros_like(kb)
    sm = c.slot_mapping.to(dev)
    lib = _lib.load()

    def wstep():
        rc = lib.qwen3_kv_write_slots_bf16(
            k.data_ptr(), _lib.strides(k, (0, 1)), v.data_ptr(), _lib.strides(v, (0, 1)),
            kb.data_ptr(), _lib.strides(kb, (0, 1, 2, 3)), vb.data_ptr(),
            _lib.strides(vb, (0, 1, 2, 3)), c.num_blocks, 0, sm.data_ptr(), sm.numel(), 8, 128,
            16, _lib.stream_of(dev))
        _lib.check(rc, "slots")

    w_wall, w_evt = time_steps(wstep, args.steps, args.warmup)
    wbytes = 8 * sum(c.lens) * 8 * 128 + 8 * sum(c.lens)
    return {"workload": f"varlen causal prefill, Qwen3-0.6B shape: 8 seqs lens={c.lens}, "
                        "16/8 heads, head_dim 128, bf16",
            "value": round(tflops, 2), "unit": "TFLOP/s", "ms_per_step": round(evt_ms, 5),
            "flops": flops,
            "roofline": {"bound": "mfma", "achieved": round(tflops, 2),
                         "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": None},
            "slot_write": {"GB/s": round(wbytes / (w_evt * 1e-3) / 1e9, 1),
                           "ms_per_step": round(w_evt, 5), "bytes": wbytes}}


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", choices=["decode", "prefill"], default=None)
    ap.add_argument("--workload", choices=["config3", "config4"], default="config3")
    ap.add_argument("--prefill-workload", choices=["config2", "steady"], default="config2",
                    help="prefill line: the Qwen3-0.6B ragged causal batch, or 8 x 4096 tokens "
                         "non-causal (steady-state rate; profiling only, with --only prefill)")
    ap.add_argument("--cpu-sample", type=int, default=64, help="sequences in the CPU baseline sample")
    ap.add_argument("--no-long-context", action="store_true",
                    help="skip the secondary long-context (B=8, up to 128k tokens) decode line")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a plain 1 GiB device copy (the known-size reference for "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args(argv)
    if args.prefill_workload != "config2" and args.only != "prefill":
        ap.error("--prefill-workload steady is a profiling line: use it with --only prefill")
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path "
              f"(asked for --gpus {args.gpus}); run with --gpus 1", file=sys.stderr)
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU (MI355X)", file=sys.stderr)
        return 1
    from qwen3_engine_from_scratch_amd import _lib

    _lib.load()
    dev = torch.device("cuda:0")
    if args.calibrate_copy:
        src = torch.ones(1 << 29, dtype=torch.bfloat16, device=dev)  # 1 GiB
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        torch.cuda.empty_cache()
    line = {"metric": METRIC, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (seeded N(0,1) q/K/V, seeded lengths and block tables)"}
    if args.only != "prefill":
        res = bench_decode(args, dev)
        gbs = res["bytes"] / (res["wall_ms"] * 1e-3) / 1e9
        ach = res["bytes"] / (res["evt_ms"] * 1e-3) / 1e9
        line.update(value=round(gbs, 1), unit="GB/s", ms_per_step=round(res["wall_ms"], 5))
        line["config"] = {"workload": res["wname"] + ", 32 q / 8 kv heads, head_dim 128, bf16, "
                          "block 16, pool 1.1x pages, random-permutation block tables",
                          "batch": len(res["lens"]), "sum_context_tokens": sum(res["lens"]),
                          "bytes_per_step": res["bytes"]}
        traffic = profiled_traffic(TRAFFIC_PROFILE) if args.workload == "config3" else None
        line["roofline"] = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS,
                            "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4),
                            "traffic": traffic, "kernel_ms": round(res["evt_ms"], 5),
                            "kernel": "paged_decode_stream_kernel + paged_decode_stream_merge_kernel "
                                      "(one decode call), HIP events on the launch stream",
                            "traffic_source": f"profiles/{TRAFFIC_PROFILE}" if traffic else None}
        if not args.no_cpu_baseline:
            line["cpu_baseline"] = cpu_baseline_decode(res, args.cpu_sample)
        del res
        torch.cuda.empty_cache()
        if args.workload == "config3" and not args.no_long_context:
            long_args = argparse.Namespace(**{**vars(args), "workload": "config4"})
            r4 = bench_decode(long_args, dev)
            line["decode_long_context"] = {
                "workload": r4["wname"] + ", 32 q / 8 kv heads, head_dim 128, bf16, block 16",
                "value": round(r4["bytes"] / (r4["evt_ms"] * 1e-3) / 1e9, 1), "unit": "GB/s",
                "ms_per_step": round(r4["evt_ms"], 5), "bytes_per_step": r4["bytes"],
                "frac_hbm_peak": round(r4["bytes"] / (r4["evt_ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
            del r4
            torch.cuda.empty_cache()
    if args.only != "decode":
        pf = bench_prefill(args, dev)
        if args.only == "prefill":
            line.update(value=pf["value"], unit=pf["unit"], ms_per_step=pf["ms_per_step"],
                        config={"workload": pf["workload"]}, roofline=pf["roofline"])
        line["prefill"] = pf
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
