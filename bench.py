"""Benchmark of the LVSA block-sparse attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config wan4x|wan6x|cog|hv|cpu]

One step = one attention call over one synthetic batch at the configuration's
full single-GPU shape, with the keyframe grid rotated by the step index
(offset = step % kfi), as in a denoising loop.  The per-offset masks and
block plans are built on the GPU before the timed region (they are built once
per denoising step and shared by every layer in a real pipeline); their cost
is reported separately.  Inputs are resident in HBM when timing starts.

Prints ONE JSON line: metric/value (effective TFLOP/s on active 128-blocks,
BASELINE's metric), ms per call, the roofline of the attention kernel
(algorithmic FLOPs per launch / HIP-event time per call on the launch stream,
vs the 2.5 PFLOP/s dense bf16 MFMA peak of MI355X; HBM traffic from a
committed rocprof counters file of the same build) and a CPU baseline (the
repository's fp32 CPU restatement timed on the host cores over a bounded
sample, extrapolated to ms per call, plus masked SDPA at the reference's CPU
configuration).
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

import longvideosparseattention_amd as lv  # noqa: E402
from longvideosparseattention_amd import hip_ops as lvops  # noqa: E402
from longvideosparseattention_amd import flops as lvflops  # noqa: E402

MFMA_BF16_PEAK_TFLOPS = 2500.0
MFMA_PEAK_TFLOPS = {"bf16": 2500.0, "f16": 2500.0, "f32": 157.3}   # MI355X dense MFMA
HBM_PEAK_GBS = 8000.0

CONFIGS = {
    # name: T, P, H, D, W, kfi, offsets, n_text, block, workload
    "wan4x": (84, 1560, 12, 128, 2, 8, list(range(8)), 0, 128,
              "Wan2.1-1.3B 4x horizon self-attention (84 latent frames x 1560 tokens)"),
    "wan6x": (121, 1560, 12, 128, 2, 8, list(range(8)), 0, 128,
              "Wan2.1-1.3B 6x horizon self-attention (121 latent frames x 1560 tokens)"),
    "cog": (13, 1350, 48, 64, 1, 4, [0], 226, 64,
            "CogVideoX-5B joint attention (226 text + 13 x 1350 video tokens)"),
    "hv": (49, 1590, 16, 128, 2, 8, list(range(8)), 256, 128,
           "HunyuanVideo-1.5 480p 1.5x dual-stream attention (49 x 1590 video + 256 text)"),
    "cpu": (9, 256, 12, 128, 1, 4, [3], 0, 64,
            "reference CPU configuration (9 latent frames x 256 tokens)"),
}


def parse(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=24)
    # warm-up calls are untimed; 16 let the clock settle (a 2 ms CogVideoX call
    # still ramps over its first ten or so)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--config", default="wan4x", choices=sorted(CONFIGS))
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU-baseline sample budget")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--dtype", choices=["bf16", "f16", "f32"], default=None,
                    help="input dtype; default bf16, and f32 for the reference's CPU configuration, which is "
                         "quoted in fp32 (fp32 inputs run the fp32 MFMA kernel)")
    ap.add_argument("--window", type=int, default=None,
                    help="override the configuration's sliding window (the Wan 6x sweep uses 1, 2, 4)")
    ap.add_argument("--head-dim", type=int, default=None, choices=[64, 96, 128, 192, 256],
                    help="override the configuration's head size (the plugin's head sizes, same geometry)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="instead of the benchmark, copy a MIB-MiB device buffer 4 times (one kernel each): "
                         "the known-size reference that scales rocprof FETCH_SIZE / WRITE_SIZE to bytes")
    return ap.parse_args(argv)


def copy_calibration(mib: int) -> int:
    """Plain device-to-device copies of a known size, for counter calibration."""
    n = mib << 20
    x = torch.ones(n, dtype=torch.uint8, device="cuda")
    y = torch.empty_like(x)
    for _ in range(4):
        y.copy_(x)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes_read": n, "copy_calibration_bytes_written": n, "launches": 4}))
    return 0


def source_hash() -> str:
    """Hash of what is compiled (the HIP sources, headers, the generated key
    loop and the build script): names the build a committed counters file was
    measured on.  The loop generator itself is left out: its output, the
    .inc, is hashed, so a comment in the generator does not rename the build."""
    import hashlib

    h = hashlib.sha256()
    pkg = os.path.join(ROOT, "longvideosparseattention_amd")
    csrc = os.path.join(pkg, "csrc")
    files = sorted(f for f in os.listdir(csrc) if f.endswith((".hip", ".h", ".inc")))
    for name in files + ["../build_lib.py", "../../include/lvsa_amd.h"]:
        with open(os.path.join(csrc, name), "rb") as f:
            h.update(name.encode() + b"\0" + f.read())
    return h.hexdigest()[:16]


def profiled_traffic(config: str):
    """HBM bytes per attention launch for `config` from the two rocprofv3
    --pmc runs summarised under profiles/ (FETCH_SIZE, WRITE_SIZE, each scaled
    by the same counter on a 1 GiB copy), used only when that file was
    measured on this build (its source_hash equals source_hash()).
    Returns (bytes or None, file, note)."""
    import glob
    import re

    here = source_hash()
    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", "*.md"))):
        with open(path) as f:
            text = f.read()
        m = re.search(r"traffic_bytes_per_launch\[" + re.escape(config) + r"\]\s*=\s*(\d+)", text)
        if not m:
            continue
        rel = os.path.relpath(path, ROOT)
        hm = re.search(r"source_hash\s*=\s*([0-9a-f]+)", text)
        if hm is None or hm.group(1) != here:
            return None, rel, f"measured on another build ({hm.group(1) if hm else 'unrecorded'} != {here})"
        return int(m.group(1)), rel, "same build"
    return None, None, "no counters file for this configuration"


def cpu_baseline(q, k, v, qt, kt, vt, meta, budget_s: float, f_block_per_call: float):
    """The fp32 CPU restatement of the call (per-frame gather + dense
    attention, the reference's lvsa_sdpa loop) on the host cores.

    A bounded sample of (head, query frame) pairs is timed and extrapolated
    linearly to the whole call by H*T / pairs; text-query rows (dense over all
    keys) are timed for one head and scaled by H.  Reported as ms per call and
    as effective TFLOP/s with the GPU line's FLOP count.  Also times fp32
    masked SDPA with the full [2304, 2304] token mask at the reference's CPU
    configuration (1 warm-up, median of 5)."""
    import torch.nn.functional as F

    from oracle import attention as oa  # CPU-baseline leg only
    from oracle import lvsa_mask as om

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    P = meta.num_patches
    T = meta.total_latent_frames
    H = q.shape[2]
    rows = [set(meta._attended_rows[f]) for f in range(T)]
    n_pairs = 0
    t0 = time.perf_counter()
    for h in range(H):
        for f in range(T):
            qs = slice(f * P, (f + 1) * P)
            parts_k = [k[:, g * P:(g + 1) * P, h:h + 1] for g in sorted(rows[f])]
            parts_v = [v[:, g * P:(g + 1) * P, h:h + 1] for g in sorted(rows[f])]
            if kt is not None:
                parts_k.append(kt[:, :, h:h + 1])
                parts_v.append(vt[:, :, h:h + 1])
            oa.dense_attention(q[:, qs, h:h + 1], torch.cat(parts_k, 1), torch.cat(parts_v, 1))
            n_pairs += 1
            if time.perf_counter() - t0 >= 0.8 * budget_s:
                break
        if time.perf_counter() - t0 >= 0.8 * budget_s:
            break
    pair_ms = 1e3 * (time.perf_counter() - t0) / n_pairs
    text_ms = 0.0
    if qt is not None:
        t1 = time.perf_counter()
        oa.text_row_attention(qt[:, :, :1], k[:, :, :1], v[:, :, :1], kt[:, :, :1], vt[:, :, :1])
        text_ms = 1e3 * (time.perf_counter() - t1) * H
    factor = H * T / n_pairs
    ms_call = pair_ms * H * T + text_ms

    # reference CPU configuration: 12 heads, D 128, 9 frames x 256, kfi 4 at step 3, window 1
    g = torch.Generator().manual_seed(0)
    cq, ck, cv = (torch.randn(1, 12, 2304, 128, generator=g) for _ in range(3))
    rel = om.build_frame_mask(9, 256, 1, 1, 4, offset=3).rows
    mask = torch.from_numpy(om.token_mask([set(r) for r in rel], 256, 2304, 2304))
    times = []
    for i in range(6):
        t1 = time.perf_counter()
        F.scaled_dot_product_attention(cq, ck, cv, attn_mask=mask)
        if i:
            times.append(1e3 * (time.perf_counter() - t1))
    sdpa_ms = sorted(times)[len(times) // 2]
    return {"value": round(f_block_per_call / (ms_call * 1e-3) / 1e12, 4), "unit": "TFLOP/s", "cores": threads,
            "kind": "port", "ms_per_call": round(ms_call, 1), "extrapolation_factor": round(factor, 2),
            "sample": f"{n_pairs} of {H * T} (head, query-frame) pairs of the same call, fp32 per-frame "
                      f"gather + dense attention, {pair_ms:.2f} ms each, x{factor:.2f} to the call"
                      + (f"; text rows timed for 1 head, x{H}" if qt is not None else ""),
            "cpu_config_masked_sdpa_ms": round(sdpa_ms, 2),
            "cpu_config_masked_sdpa": "fp32 F.scaled_dot_product_attention, 12 heads, [2304, 2304] token mask "
                                      "(9 frames x 256, kfi 4 at step 3, window 1), median of 5 after 1 warm-up"}


def main(argv=None) -> int:
    args = parse(argv)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs the LVSA hot path on ONE GPU; multi-GPU runs are not part of it "
              "(the design notes describe how the path would shard over heads).", file=sys.stderr)
        return 2
    if args.copy_calibration:
        return copy_calibration(args.copy_calibration)
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    dev = torch.device("cuda", 0)
    T, P, H, D, W, kfi, offsets, n_text, block, workload = CONFIGS[args.config]
    if args.window is not None:
        W = args.window
        workload += f", window +-{W}"
    if args.head_dim is not None and args.head_dim != D:
        D = args.head_dim
        workload += f", head size {D}"
    N = T * P
    dname = args.dtype or ("f32" if args.config == "cpu" else "bf16")
    dt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[dname]
    peak = MFMA_PEAK_TFLOPS[dname]

    # Synthetic inputs: one CPU generator, fp32 randn in order q, k, v, text q, k, v.
    g = torch.Generator().manual_seed(args.seed)
    q32, k32, v32 = (torch.randn(1, N, H, D, generator=g) for _ in range(3))
    qt32 = kt32 = vt32 = None
    if n_text:
        qt32, kt32, vt32 = (torch.randn(1, n_text, H, D, generator=g) for _ in range(3))
    q, k, v = (x.to(dt).to(dev) for x in (q32, k32, v32))
    qt = kt = vt = None
    if n_text:
        qt, kt, vt = (x.to(dt).to(dev) for x in (qt32, kt32, vt32))

    # Per-offset metadata + plans (device), built and timed outside the step loop.
    metas = {}
    build_ms = []
    for off in offsets:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        m = lv.LVSAMetadata.build(total_latent_frames=T, num_patches=P, window_size=W, n_first_frames=1,
                                  key_frame_interval=kfi, rank=0, world=1, keyframe_offset=off)
        m.full_plan(dev, N, N, n_text, n_text, D, dt)
        torch.cuda.synchronize()
        build_ms.append(1e3 * (time.perf_counter() - t0))
        metas[off] = m
    flops = {off: lvflops.attention_flops(metas[off], dev, block, H, D, n_text) for off in offsets}

    def step(i):
        m = metas[offsets[i % len(offsets)]]
        if n_text:
            return lv.lvsa_attention(q, k, v, m, k_text=kt, v_text=vt, q_text=qt)
        return lv.lvsa_attention(q, k, v, m)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    # events on the stream the kernels are launched on (torch's current
    # stream), one between consecutive calls: per-call times without a host
    # synchronisation inside the timed region
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    t0 = time.perf_counter()
    evs[0].record()
    for i in range(args.steps):
        step(i)
        evs[i + 1].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    call_ms = [evs[i].elapsed_time(evs[i + 1]) for i in range(args.steps)]
    ev_ms = evs[0].elapsed_time(evs[-1]) / args.steps
    ev_median = sorted(call_ms)[args.steps // 2] if args.steps % 2 else \
        0.5 * sum(sorted(call_ms)[args.steps // 2 - 1:args.steps // 2 + 1])
    ms = 1e3 * wall / args.steps
    fb = sum(flops[offsets[i % len(offsets)]][0] for i in range(args.steps))
    fx = sum(flops[offsets[i % len(offsets)]][1] for i in range(args.steps))
    value = fb / wall / 1e12
    achieved = fb / (ev_ms * 1e-3 * args.steps) / 1e12
    per_call_tf = sorted(flops[offsets[i % len(offsets)]][0] / (call_ms[i] * 1e-3) / 1e12 for i in range(args.steps))
    achieved_median = per_call_tf[args.steps // 2] if args.steps % 2 else \
        0.5 * (per_call_tf[args.steps // 2 - 1] + per_call_tf[args.steps // 2])
    bytes_per_call = 4 * (N + n_text) * H * D * 2
    tag = args.config + ("" if args.window is None else f"_w{W}") + (
        "" if args.head_dim is None or args.head_dim == CONFIGS[args.config][3] else f"_d{D}")
    traffic, traffic_src, traffic_note = profiled_traffic(tag)
    # every 16-bit head size runs the single-stream kernel on these geometries
    # (D = 192 in its dual-wide map, 256 in its wide map); LVSA_ATTN_KERNEL=pp selects the
    # ping-pong kernel (D <= 128) or the 4-wave kernel (D >= 192)
    kernel = "attn_fwd_stream_kernel"
    if os.environ.get("LVSA_ATTN_KERNEL") == "pp":
        kernel = "attn_fwd_pp_kernel" if D <= 128 else "attn_fwd_kernel"
    if dname == "f32":
        kernel = "attn_fwd_f32_kernel"

    line = {
        "metric": f"block-sparse attn ms/call + effective TFLOP/s (% {'fp32' if dname == 'f32' else 'bf16'} "
                  "MFMA peak), " + {"wan4x": "Wan 4x shape"}.get(args.config, args.config + " shape"),
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        # median of the per-call HIP-event times (the keyframe offset rotates,
        # so calls differ in work by a few percent)
        "ms_per_call_median": round(ev_median, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dname,
        "data": f"synthetic: seeded N(0,1) q/k/v, {dname}, RoPE-free; keyframe offset = step % kfi",
        "config": {"workload": workload, "T": T, "P": P, "heads": H, "head_dim": D, "window": W,
                   "kfi": kfi, "n_first": 1, "offsets": offsets, "text_tokens": n_text, "block": block,
                   "batch": 1, "parallelism": "single GPU"},
        "pct_bf16_mfma_peak": round(100 * value / MFMA_BF16_PEAK_TFLOPS, 2),
        "pct_mfma_peak": round(100 * value / peak, 2),      # of the MFMA peak of the input dtype
        "tflops_token_exact": round(fx / wall / 1e12, 2),
        "gflop_per_call_block": round(fb / args.steps / 1e9, 1),
        "hbm_gbs_algorithmic": round(bytes_per_call / (ms * 1e-3) / 1e9, 1),
        # per offset, warm (median over offsets after the first); the first
        # build also pays the one-time library load and code-object upload
        "mask_and_plan_build_ms": round(sorted(build_ms[1:] or build_ms)[len(build_ms[1:] or build_ms) // 2], 3),
        "mask_and_plan_first_build_ms": round(build_ms[0], 3),
        # achieved = block FLOPs / the HIP-event span of the timed calls on the
        # launch stream (the attention kernel, plus the text merge kernel
        # where text tiles are split); rocprof kernel averages: profiles/
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": peak,
                     "unit": "TFLOP/s", "frac": round(achieved / peak, 4), "traffic": traffic,
                     "traffic_source": traffic_src, "traffic_note": traffic_note, "kernel": kernel,
                     "event_ms_per_call": round(ev_ms, 4), "event_ms_per_call_median": round(ev_median, 4),
                     "event_ms_per_call_min_max": [round(min(call_ms), 4), round(max(call_ms), 4)],
                     "achieved_median": round(achieved_median, 2), "build": source_hash()},
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(q.float().cpu(), k.float().cpu(), v.float().cpu(),
                                            None if qt is None else qt.float().cpu(),
                                            None if kt is None else kt.float().cpu(),
                                            None if vt is None else vt.float().cpu(),
                                            metas[offsets[0]], args.cpu_seconds, fb / args.steps)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
