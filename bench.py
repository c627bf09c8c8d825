"""Benchmark: paged INT8 decode attention, B8 H32 S4096 D128 (BASELINE.json metric) on one GPU.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

One step = one ``paged_quant_attention_triton`` call over one batch (8 requests x 32
heads x 4096 cached tokens, 16-token pages, fp16 query, INT8 K/V with fp32 scale and
int16 zero point per page and head).  Inputs are synthetic, resident in HBM before
timing, and rotated over 3 independent sets (3 x 269 MB) so the 256 MB Infinity
Cache cannot serve a step from the previous one.  Prints ONE JSON line.

``value`` = algorithmic bytes per step / measured time per step (GB/s).
Algorithmic bytes = int8 K+V (2*sum(L)*H*D) + fp32 scale and int16 zero per page and
head for K and V + int64 table entries + int64 lengths + fp16 q and output.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "decode-attn µs/step + achieved HBM GB/s (% of peak), paged INT8 B8 H32 s4096 d128"
PEAK_GBPS = 8000.0  # MI355X HBM3E
B, H, S, D, PAGE = 8, 32, 4096, 128, 16
ROTATE = 3
# Rotated input sets must together exceed the 256 MiB MALL (last-level cache) twice over, so a
# timed step cannot be served from what an earlier step left there.
MALL_BYTES = 256 << 20


def rotation_sets(set_bytes: int) -> int:
    """Input sets to rotate for a workload of `set_bytes` per step: at least ROTATE, and enough
    that they hold at least 2 x MALL_BYTES together."""

    return max(ROTATE, math.ceil(2 * MALL_BYTES / max(1, set_bytes)))
PMC_SUMMARY = ROOT / "profiles" / "paged_decode_b8h32s4096d128_pmc.json"


def algorithmic_bytes(lengths, heads: int, head_dim: int, page: int, q_bytes: int = 2, idx_bytes: int = 8,
                      quant_block: int | None = None, param_bytes: int = 6) -> int:
    """param_bytes per quant block and tensor: fp32 scale + int16 zero (INT8), fp32 scale (FP8)."""

    pages = sum(math.ceil(L / page) for L in lengths)
    blocks = sum(math.ceil(L / (quant_block or page)) for L in lengths)
    kv = 2 * sum(lengths) * heads * head_dim
    params = 2 * blocks * heads * param_bytes
    table = pages * idx_bytes
    return kv + params + table + 8 * len(lengths) + 2 * len(lengths) * heads * head_dim * q_bytes


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=300)
    ap.add_argument("--warmup", type=int, default=1000)
    ap.add_argument("--no-cpu-baseline", action="store_true", help="skip the CPU oracle timing")
    ap.add_argument("--only", default="", help="--mode shapes: comma-separated shape names to run")
    ap.add_argument("--layout", default="contiguous", choices=["contiguous", "shuffled", "interleaved"])
    ap.add_argument("--mode", default="full", choices=["full", "paged", "copy", "readbw", "serving", "shapes", "tree"],
                    help="full: the JSON line; paged: only the timed paged steps (for rocprofv3); "
                         "copy: a plain 256 MiB device copy, to calibrate rocprofv3 byte counters; "
                         "readbw: the library's plain streaming read of 256 MiB (the practical read ceiling); "
                         "serving: only the 64-request serving decode step; shapes: the SHAPES table; "
                         "tree: tree verification for 1-16 draft nodes")
    return ap.parse_args()


def copy_calibration(torch, steps: int) -> int:
    """`steps` copies of 256 MiB (read 256 MiB + write 256 MiB each) with torch's copy kernel."""

    n = 256 * 1024 * 1024 // 4
    src = torch.randn(n, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"mode": "copy", "bytes_read_per_copy": n * 4, "bytes_written_per_copy": n * 4,
                      "copies": steps}), flush=True)
    return 0


def make_inputs(torch, fa, dev, seed: int, layout: str):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    q = torch.randn((B, H, D), generator=g, device=dev, dtype=torch.float16)
    k = torch.randn((B, H, S, D), generator=g, device=dev, dtype=torch.float16)
    v = torch.randn((B, H, S, D), generator=g, device=dev, dtype=torch.float16)
    cache = fa.PagedKVCache.from_dense(k, v, block_size=PAGE, block_table_pattern=layout, layout_seed=seed)
    kq = fa.quantize_int8_per_block(k, PAGE)
    vq = fa.quantize_int8_per_block(v, PAGE)
    del k, v
    return q, cache, kq, vq


STREAM_READ_BYTES = 256 << 20
STREAM_READ_BLOCKS = 2048


def stream_read_ceiling(torch, dev, steps: int = 60) -> dict:
    """Practical HBM read ceiling: the library's plain streaming-read kernel (`fs_stream_read`,
    16-byte loads, grid-stride) over 3 rotated 256 MiB buffers, like the decode's rotated
    inputs; mean of `steps` launches on torch's current stream."""

    from flashspec_amd import _lib

    lib = _lib.require()
    bufs = [torch.full((STREAM_READ_BYTES,), i + 1, dtype=torch.uint8, device=dev) for i in range(ROTATE)]
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    stream = _lib.stream_ptr(dev)

    def read(i):
        _lib.check(lib.fs_stream_read(bufs[i % ROTATE].data_ptr(), STREAM_READ_BYTES, sink.data_ptr(),
                                      STREAM_READ_BLOCKS, stream))

    ms = time_loop(torch, read, steps, 6)
    del bufs
    return {"kernel": "stream_read_kernel", "bytes_per_launch": STREAM_READ_BYTES, "rotated_buffers": ROTATE,
            "workgroups": STREAM_READ_BLOCKS, "us": round(ms * 1e3, 2),
            "GBps": round(STREAM_READ_BYTES / (ms * 1e-3) / 1e9, 1)}


# Untimed calls of the step itself, for at least this long, before the counted warm-up: the
# GPU's clocks take tens to hundreds of milliseconds of sustained load to settle.  Measured at
# the metric shape on one box, the first timed loop read 49.2-49.9 us after 30 warm-up steps
# (1.4 ms) and 46.8-47.0 us after 1000 or 3000; with 0.1 s of settle and 5 warm-up steps, the
# first shape of `--mode shapes` still read 46.4 us where the full line read 43.1 us.
SETTLE_S = 0.25


def settle(torch, fn, seconds: float = SETTLE_S) -> int:
    """Calls fn(i) in batches of 20 until `seconds` of wall time have passed; returns the count."""

    torch.cuda.synchronize()
    t0, n = time.perf_counter(), 0
    while time.perf_counter() - t0 < seconds:
        for _ in range(20):
            fn(n)
            n += 1
        torch.cuda.synchronize()
    return n


def time_loop(torch, fn, steps: int, warmup: int) -> float:
    """Mean ms per call over `steps` calls bracketed by synchronize + events, after `settle`
    and `warmup` untimed calls."""

    settle(torch, fn)
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        fn(i)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def kernel_durations_us(torch, fn, calls: int) -> list[float]:
    """Per-launch duration: an event pair around each call on the launching stream."""

    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(calls)]
    for i, (a, b) in enumerate(evs):
        a.record()
        fn(i)
        b.record()
    torch.cuda.synchronize()
    return [a.elapsed_time(b) * 1e3 for a, b in evs]


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_run(fn, threads: int, repeats: int) -> tuple[float, int]:
    """Median seconds of `repeats` timed calls after one warm-up call, on `threads` torch threads."""

    import torch

    torch.set_num_threads(threads)
    fn()
    times = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), repeats


def cpu_baseline(torch, fa, dev) -> dict:
    """The reference's CPU path timed on this host: its PyTorch op sequence (dequantize K/V to dense
    float32, einsum, length mask, softmax, einsum, cast; reference attention.py:124-223), which is
    this package's portable path (`flashspec_amd.attention`), on the same synthetic workload as the
    GPU line.  All cores (`torch.set_num_threads(len(os.sched_getaffinity(0)))`) and one thread;
    `perf_counter`, one warm-up call, median of the repeats.

    `value`: the metric workload (paged B8 H32 S4096 D128, whole-store dequantize and gather as
    the reference's `paged_quant_attention` does) on all cores.  Also: C1 (fused B4 S2048, the
    primary CPU comparator) on all cores and on one thread, and the metric workload on one thread
    over a one-request sample (one request's pool; the reference path's cost is linear in it).
    The int8 stores are made by this library's GPU quantizer, which is bit-identical to the CPU
    path (tested), then copied to host memory; only the attention calls are timed."""

    threads = len(os.sched_getaffinity(0))
    saved = torch.get_num_threads()
    g = torch.Generator().manual_seed(0)

    def paged_inputs(b):
        q = torch.randn((b, H, D), generator=g).to(torch.float16)
        k = torch.randn((b, H, S, D), generator=g).to(torch.float16)
        v = torch.randn((b, H, S, D), generator=g).to(torch.float16)
        c = fa.PagedKVCache.from_dense(k.to(dev), v.to(dev), block_size=PAGE)
        cpu = fa.PagedKVCache(
            k_quant=fa.QuantizedTensor(*(t.cpu() for t in (c.k_quant.values, c.k_quant.scale, c.k_quant.zero_point)),
                                       c.k_quant.block_size, c.k_quant.original_shape),
            v_quant=fa.QuantizedTensor(*(t.cpu() for t in (c.v_quant.values, c.v_quant.scale, c.v_quant.zero_point)),
                                       c.v_quant.block_size, c.v_quant.original_shape),
            block_table=c.block_table.cpu(), lengths=c.lengths.cpu(), block_size=PAGE, max_seq_len=S)
        return q, cpu

    try:
        c1_b, c1_s = 4, 2048
        q1 = torch.randn((c1_b, H, D), generator=g).to(torch.float16)
        k1 = torch.randn((c1_b, H, c1_s, D), generator=g).to(torch.float16)
        v1 = torch.randn((c1_b, H, c1_s, D), generator=g).to(torch.float16)
        kq, vq = (fa.quantize_int8_per_block(x.to(dev), PAGE) for x in (k1, v1))
        kq, vq = (fa.QuantizedTensor(x.values.cpu(), x.scale.cpu(), x.zero_point.cpu(), x.block_size,
                                     x.original_shape) for x in (kq, vq))
        del k1, v1
        c1_bytes = algorithmic_bytes([c1_s] * c1_b, H, D, PAGE)
        c1_all, n1 = _median_run(lambda: fa.fused_dequant_attention(q1, kq, vq), threads, 5)
        c1_one, _ = _median_run(lambda: fa.fused_dequant_attention(q1, kq, vq), 1, 5)
        del kq, vq
        qm, cm = paged_inputs(B)
        m_all, nm = _median_run(lambda: fa.paged_quant_attention(qm, cm), threads, 5)
        del qm, cm
        qs, cs = paged_inputs(1)
        m_one, ns = _median_run(lambda: fa.paged_quant_attention(qs, cs), 1, 3)
        del qs, cs
    finally:
        torch.set_num_threads(saved)
    m_bytes = algorithmic_bytes([S] * B, H, D, PAGE)
    s_bytes = algorithmic_bytes([S], H, D, PAGE)
    return {
        "value": round(m_bytes / m_all / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
        "sample": f"the reference's torch-CPU paged path (flashspec_amd.attention.paged_quant_attention: "
                  f"whole-store dequantize, gather, einsum, mask, softmax, einsum) on the full metric workload "
                  f"B{B} H{H} S{S} D{D}, {threads} threads, median of {nm} after 1 warm-up: "
                  f"{m_all * 1e3:.1f} ms per step",
        "us_per_step": round(m_all * 1e6, 1),
        "cpu_model": cpu_model(), "torch": torch.__version__, "threads": threads,
        "c1_fused": {"workload": f"fused B{c1_b} H{H} S{c1_s} D{D} (C1), reference torch-CPU fused path",
                     "all_cores_ms": round(c1_all * 1e3, 2), "all_cores_gbps": round(c1_bytes / c1_all / 1e9, 3),
                     "one_thread_ms": round(c1_one * 1e3, 2), "one_thread_gbps": round(c1_bytes / c1_one / 1e9, 3),
                     "repeats": n1},
        "metric_one_thread": {"sample": f"1 of the {B} requests (its own page pool), B1 H{H} S{S} D{D}",
                              "ms": round(m_one * 1e3, 1), "gbps": round(s_bytes / m_one / 1e9, 3),
                              "repeats": ns},
    }


SERVE_B, SERVE_LO, SERVE_HI = 64, 128, 16384


def serving_step_bench(torch, fa, dev, steps: int, warmup: int) -> dict:
    """Serving decode step at scale: 64 requests, lengths ~ U[128, 16384] (seeded CPU draw),
    fragmented shuffled page pool, one fp16 token appended per request per step and paged
    attention over the updated cache: ``DecodeBatch.step``, device-resident table and lengths.
    At this size (2048 rows, several rounds of workgroups per CU) the step is two launches, the
    append kernel and then the decode (requests dispatched longest first); the one-launch form,
    with the append inside the decode kernel, serves grids of one round of workgroups."""

    from flashspec_amd.serving import DecodeBatch, build_request_pool

    g = torch.Generator().manual_seed(0)
    lengths = torch.randint(SERVE_LO, SERVE_HI + 1, (SERVE_B,), generator=g).tolist()
    total = warmup + steps
    alloc, rids = build_request_pool(lengths, heads=H, head_dim=D, block_size=PAGE, headroom_tokens=total + 1,
                                     seed=0, device=dev, dtype=torch.float16)
    batch = DecodeBatch(alloc, rids, max_new_tokens=total, reserve_steps=total)
    gd = torch.Generator(device=dev)
    gd.manual_seed(1)
    n_in = 4
    qs = [torch.randn((SERVE_B, H, D), generator=gd, device=dev, dtype=torch.float16) for _ in range(n_in)]
    ks = [torch.randn((SERVE_B, H, 1, D), generator=gd, device=dev, dtype=torch.float16) for _ in range(n_in)]
    vs = [torch.randn((SERVE_B, H, 1, D), generator=gd, device=dev, dtype=torch.float16) for _ in range(n_in)]
    # settle the clocks with attention-only calls: a step appends, so it cannot repeat freely
    settle(torch, lambda i: batch.attend(qs[i % n_in]))
    for i in range(warmup):
        batch.step(qs[i % n_in], ks[i % n_in], vs[i % n_in])
    torch.cuda.synchronize()
    len0 = list(batch.host_lengths)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        batch.step(qs[i % n_in], ks[i % n_in], vs[i % n_in])
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    _, stats = batch.attend(qs[0], return_stats=True)
    # attention over lengths len0+1 .. len0+steps, averaged; the append reads and writes one
    # K and one V page (int8 + scale + zero) per request and head and reads the new token
    mean_len = [L + (steps + 1) / 2 for L in len0]
    attn_bytes = algorithmic_bytes([round(L) for L in mean_len], H, D, PAGE)
    append_bytes = 2 * SERVE_B * H * (2 * (PAGE * D + 6) + D * 2)
    nbytes = attn_bytes + append_bytes
    batch.close()
    res = {
        "workload": f"serving decode step: B{SERVE_B} ragged lengths ~U[{SERVE_LO},{SERVE_HI}] (seeded), H{H} D{D}, "
                    f"{PAGE}-token pages in a shuffled pool, append one fp16 token per request + paged attention",
        "sum_lengths": sum(len0), "us_per_step": round(ms * 1e3, 2),
        "algorithmic_bytes_per_step": nbytes, "gbps": round(nbytes / (ms * 1e-3) / 1e9, 1),
        "pct_of_peak": round(100.0 * nbytes / (ms * 1e-3) / 1e9 / PEAK_GBPS, 1),
        "num_splits": stats.get("num_splits"), "steps": steps, "warmup": warmup,
    }
    del batch, alloc
    torch.cuda.empty_cache()
    return res


def quantize_bench(torch, fa, dev, calls: int = 30) -> dict:
    """quantize_int8_per_block of one fp16 K tensor of the metric workload ([8, 32, 4096, 128],
    16-token blocks), input resident in HBM; bytes = fp16 read + int8 write + scale/zero write.
    Beside it, the practical ceiling of that traffic on the same GPU: a streaming 2:1 copy of
    the same tensor (`fs_stream_copy_half`)."""

    from flashspec_amd import _lib

    g = torch.Generator(device=dev)
    g.manual_seed(5)
    xs = [torch.randn((B, H, S, D), generator=g, device=dev, dtype=torch.float16) for _ in range(2)]
    ms = time_loop(torch, lambda i: fa.quantize_int8_per_block(xs[i % 2], PAGE), calls, 3)
    groups = B * H * (S // PAGE)
    nbytes = B * H * S * D * (2 + 1) + groups * 6
    # the same traffic with no arithmetic: fs_stream_copy_half reads the fp16 tensor and writes
    # half as many bytes, best of a few grid sizes
    lib = _lib.require()
    dst = torch.empty(B * H * S * D, dtype=torch.int8, device=dev)
    src_bytes = xs[0].numel() * 2
    stream = _lib.stream_ptr(dev)
    best = None
    for blocks in (2048, 4096, 8192):
        cms = time_loop(torch, lambda i: _lib.check(lib.fs_stream_copy_half(
            xs[i % 2].data_ptr(), src_bytes, dst.data_ptr(), blocks, stream)), calls, 3)
        if best is None or cms < best[0]:
            best = (cms, blocks)
    copy_bytes = src_bytes + src_bytes // 2
    copy_gbps = copy_bytes / (best[0] * 1e-3) / 1e9
    del xs, dst
    gbps = nbytes / (ms * 1e-3) / 1e9
    return {"workload": f"quantize_int8_per_block fp16 [{B}, {H}, {S}, {D}], block {PAGE}",
            "us_per_call": round(ms * 1e3, 2), "algorithmic_bytes": nbytes,
            "gbps": round(gbps, 1), "pct_of_peak": round(100 * gbps / PEAK_GBPS, 1),
            "copy_ceiling": {"kernel": "stream_copy_half_kernel", "bytes": copy_bytes, "us": round(best[0] * 1e3, 2),
                             "gbps": round(copy_gbps, 1), "workgroups": best[1]},
            "frac_of_copy_ceiling": round(gbps / copy_gbps, 4)}


def page_quantize_bench(torch, fa, dev, calls: int = 30) -> dict:
    """``PagedKVCache.from_dense``'s page quantizer (``fs_quantize_pages_i8``, one launch per tensor)
    on one fp16 K tensor of the metric workload ([8, 32, 4096, 128] into 2048 16-token pages), in the
    contiguous and the shuffled page order, input resident in HBM and rotated over two tensors;
    bytes = fp16 read + int8 write + scale/zero write.  Beside it the same 2:1 copy ceiling as the
    blocks quantizer's (`fs_stream_copy_half` over the same tensor, best grid)."""

    from flashspec_amd import _lib

    lib = _lib.require()
    g = torch.Generator(device=dev)
    g.manual_seed(6)
    xs = [torch.randn((B, H, S, D), generator=g, device=dev, dtype=torch.float16) for _ in range(2)]
    pages = B * (S // PAGE)
    values = torch.empty((pages, H, 1, PAGE, D), dtype=torch.int8, device=dev)
    scale = torch.empty((pages, H, 1, 1, 1), dtype=torch.float32, device=dev)
    zero = torch.empty((pages, H, 1, 1, 1), dtype=torch.int16, device=dev)
    stream = _lib.stream_ptr(dev)
    gp = torch.Generator(device=dev)
    gp.manual_seed(0)
    perm = torch.randperm(pages, generator=gp, device=dev)
    nbytes = B * H * S * D * (2 + 1) + pages * H * 6
    out = {"workload": f"fs_quantize_pages_i8 fp16 [{B}, {H}, {S}, {D}] -> {pages} pages of {PAGE} tokens",
           "algorithmic_bytes": nbytes}
    for name, src in (("contiguous", None), ("shuffled", perm)):
        def call(i, src=src):
            _lib.check(lib.fs_quantize_pages_i8(
                xs[i % 2].data_ptr(), 1, B, H, S, D, PAGE, _lib.ptr(src), pages, values.data_ptr(),
                scale.data_ptr(), zero.data_ptr(), stream))
        ms = time_loop(torch, call, calls, 3)
        gbps = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"us_per_call": round(ms * 1e3, 2), "gbps": round(gbps, 1),
                     "pct_of_peak": round(100 * gbps / PEAK_GBPS, 1)}
    dst = torch.empty(B * H * S * D, dtype=torch.int8, device=dev)
    src_bytes = xs[0].numel() * 2
    best = None
    for blocks in (2048, 4096, 8192):
        cms = time_loop(torch, lambda i: _lib.check(lib.fs_stream_copy_half(
            xs[i % 2].data_ptr(), src_bytes, dst.data_ptr(), blocks, stream)), calls, 3)
        if best is None or cms < best[0]:
            best = (cms, blocks)
    copy_gbps = (src_bytes + src_bytes // 2) / (best[0] * 1e-3) / 1e9
    out["copy_ceiling"] = {"kernel": "stream_copy_half_kernel", "us": round(best[0] * 1e3, 2),
                           "gbps": round(copy_gbps, 1), "workgroups": best[1]}
    for name in ("contiguous", "shuffled"):
        out[name]["frac_of_copy_ceiling"] = round(out[name]["gbps"] / copy_gbps, 4)
    del xs, dst, values, scale, zero
    return out


def c2_configured_bench(torch, fa, sets, steps: int, warmup: int, fused_ms: float, nbytes: int) -> dict:
    """BASELINE config 2 as configured: the contiguous (fused) decode B8 H32 S4096 D128 with
    FLASHSPEC_NUM_SPLITS=4 (the reference's own published point, triton_fused split 4), over the
    metric's rotated input sets, beside the planner's plan on the same data (`fused_ms`)."""

    old = os.environ.get("FLASHSPEC_NUM_SPLITS")
    os.environ["FLASHSPEC_NUM_SPLITS"] = "4"
    try:
        def step(i):
            q, _, kq, vq = sets[i % ROTATE]
            return fa.fused_dequant_attention_triton(q, kq, vq)

        _, st = fa.fused_dequant_attention_triton(sets[0][0], sets[0][2], sets[0][3], return_stats=True)
        ms = time_loop(torch, step, steps, warmup)
    finally:
        if old is None:
            del os.environ["FLASHSPEC_NUM_SPLITS"]
        else:
            os.environ["FLASHSPEC_NUM_SPLITS"] = old
    gbps = nbytes / (ms * 1e-3) / 1e9
    return {"workload": f"fused INT8 decode B{B} H{H} S{S} D{D}, FLASHSPEC_NUM_SPLITS=4, {ROTATE} rotated sets",
            "us_per_step": round(ms * 1e3, 2), "gbps": round(gbps, 1), "pct_of_peak": round(100 * gbps / PEAK_GBPS, 1),
            "num_splits": st.get("num_splits"), "waves_per_workgroup": st.get("num_warps"),
            "planner_us_per_step": round(fused_ms * 1e3, 2), "vs_planner": round(ms / fused_ms, 4)}


# Shapes beyond the metric workload: (name, batch, heads, seq, head_dim, page, quant block, q dtype, lengths
# [, format [, page layout]]); quant block 1 = symmetric absmax INT8 with one scale per token
# (quantize_int8_symmetric_per_token), or one FP8 scale per token with format "fp8"; format
# "channel" = per-channel affine INT8 (quantize_int8_per_channel); page layout = from_dense's
# block_table_pattern (contiguous by default).
SHAPES = [
    ("metric", 8, 32, 4096, 128, 16, 16, "float16", None),
    ("c1_affine", 4, 32, 2048, 128, 16, 16, "float16", None),
    ("c3_s2048", 8, 32, 2048, 128, 16, 16, "float16", None),
    ("c4_descending_tail", 16, 32, 4096, 128, 16, 16, "float16", [4096 - 256 * i - 7 for i in range(16)]),
    ("c4_shuffled", 16, 32, 4096, 128, 16, 16, "float16", [4096 - 256 * i for i in range(16)], "int8", "shuffled"),
    ("c4_interleaved", 16, 32, 4096, 128, 16, 16, "float16", [4096 - 256 * i for i in range(16)], "int8",
     "interleaved"),
    ("head_dim_64", 8, 32, 4096, 64, 16, 16, "float16", None),
    ("head_dim_256", 8, 32, 4096, 256, 16, 16, "float16", None),
    ("page_32_quant_16", 8, 32, 4096, 128, 32, 16, "float16", None),
    ("q_bfloat16", 8, 32, 4096, 128, 16, 16, "bfloat16", None),
    ("q_float32", 8, 32, 4096, 128, 16, 16, "float32", None),
    ("block_32", 8, 32, 4096, 128, 32, 32, "float16", None),
    ("page_64_quant_32", 8, 32, 4096, 128, 64, 32, "float16", None),
    ("head_dim_96", 8, 32, 4096, 96, 16, 16, "float16", None),
    ("head_dim_192", 8, 32, 4096, 192, 16, 16, "float16", None),
    ("block_8", 8, 32, 4096, 128, 8, 8, "float16", None),
    ("page_16_quant_8", 8, 32, 4096, 128, 16, 8, "float16", None),
    ("head_dim_40", 8, 32, 4096, 40, 16, 16, "float16", None),
    ("head_dim_120", 8, 32, 4096, 120, 16, 16, "float16", None),
    ("head_dim_36", 8, 32, 4096, 36, 16, 16, "float16", None),
    ("head_dim_100", 8, 32, 4096, 100, 16, 16, "float16", None),
    ("q_bfloat16_head_dim_100", 8, 32, 4096, 100, 16, 16, "bfloat16", None),
    ("head_dim_34_generic", 8, 32, 4096, 34, 16, 16, "float16", None),
    ("batch_1_splitk", 1, 32, 16384, 128, 16, 16, "float16", None),
    ("c1_symmetric_per_token", 4, 32, 2048, 128, 16, 1, "float16", None),
    ("c2_symmetric_per_token", 8, 32, 4096, 128, 16, 1, "float16", None),
    ("metric_fp8", 8, 32, 4096, 128, 16, 16, "float16", None, "fp8"),
    ("head_dim_64_fp8", 8, 32, 4096, 64, 16, 16, "float16", None, "fp8"),
    ("q_bfloat16_fp8", 8, 32, 4096, 128, 16, 16, "bfloat16", None, "fp8"),
    ("fp8_per_token", 8, 32, 4096, 128, 16, 1, "float16", None, "fp8"),
    ("per_channel_block_16", 8, 32, 4096, 128, 16, 16, "float16", None, "channel"),
    ("per_channel_block_32", 8, 32, 4096, 128, 32, 32, "float16", None, "channel"),
    ("per_channel_block_64", 8, 32, 4096, 128, 64, 64, "float16", None, "channel"),
    ("per_channel_block_128", 8, 32, 4096, 128, 128, 128, "float16", None, "channel"),
    ("per_channel_head_dim_64_block_64", 8, 32, 4096, 64, 64, 64, "float16", None, "channel"),
    ("per_channel_head_dim_256_block_64", 8, 32, 2048, 256, 64, 64, "float16", None, "channel"),
]


def paged_from_blocks(torch, fa, k, v, page: int, qb: int, lengths):
    """Contiguous-layout page store whose pages hold page // qb quant blocks (page != quant block):
    physical page b * pages_per_seq + j = logical page j of request b."""

    b, h, s, d = k.shape
    nbps = (s + page - 1) // page
    per = page // qb

    def pages(x):
        xq = fa.quantize_int8_per_block(torch.nn.functional.pad(x, (0, 0, 0, nbps * page - s)), qb)
        vals = xq.values.reshape(b, h, nbps, per, qb, d).permute(0, 2, 1, 3, 4, 5).reshape(b * nbps, h, per, qb, d)
        sc = xq.scale.reshape(b, h, nbps, per).permute(0, 2, 1, 3).reshape(b * nbps, h, per, 1, 1)
        zp = xq.zero_point.reshape(b, h, nbps, per).permute(0, 2, 1, 3).reshape(b * nbps, h, per, 1, 1)
        return fa.QuantizedTensor(vals.contiguous(), sc.contiguous(), zp.contiguous(), qb, (b * nbps, h, page, d))

    table = torch.arange(b * nbps, dtype=torch.int64, device=k.device).reshape(b, nbps)
    lens = lengths if lengths is not None else torch.full((b,), s, dtype=torch.int64, device=k.device)
    return fa.PagedKVCache(k_quant=pages(k), v_quant=pages(v), block_table=table, lengths=lens, block_size=page,
                           max_seq_len=s)


def shapes_bench(torch, fa, dev, steps: int, warmup: int, only=None) -> list[dict]:
    """Paged and contiguous decode over the SHAPES table (or the shapes named in `only`), with
    `rotation_sets` input sets each (at least 3, and at least 2 x the MALL together); prints one
    JSON object per shape."""

    out = []
    for name, b, h, s, d, page, qb, qdt, lens, *rest in SHAPES:
        if only and name not in only:
            continue
        fmt = rest[0] if rest else "int8"
        layout = rest[1] if len(rest) > 1 else "contiguous"
        g = torch.Generator(device=dev)
        g.manual_seed(11)
        qdtype = getattr(torch, qdt)
        lengths = lens or [s] * b
        nbytes = algorithmic_bytes(lengths, h, d, page, q_bytes=torch.finfo(qdtype).bits // 8, quant_block=qb,
                                   param_bytes={"fp8": 4, "channel": 6 * d}.get(fmt, 6))
        n_sets = rotation_sets(nbytes)
        sets = []
        for _ in range(n_sets):
            q = torch.randn((b, h, d), generator=g, device=dev, dtype=torch.float16).to(qdtype)
            k = torch.randn((b, h, s, d), generator=g, device=dev, dtype=torch.float16)
            v = torch.randn((b, h, s, d), generator=g, device=dev, dtype=torch.float16)
            lt = None if lens is None else torch.tensor(lens, dtype=torch.int64, device=dev)
            if fmt == "channel":
                cache = fa.PagedKVCache.from_dense(k, v, block_size=page, lengths=lt, kv_format="affine_channel")
                kq, vq = fa.quantize_int8_per_channel(k, qb), fa.quantize_int8_per_channel(v, qb)
            elif fmt == "fp8":
                if qb == 1:
                    pk = fa.PagedKVCache._physical_pages(k, page, None)
                    pv = fa.PagedKVCache._physical_pages(v, page, None)
                    nbps = (s + page - 1) // page
                    cache = fa.PagedKVCache(
                        k_quant=fa.quantize_fp8_per_block(pk, 1), v_quant=fa.quantize_fp8_per_block(pv, 1),
                        block_table=torch.arange(b * nbps, dtype=torch.int64, device=dev).reshape(b, nbps),
                        lengths=lt if lt is not None else torch.full((b,), s, dtype=torch.int64, device=dev),
                        block_size=page, max_seq_len=s)
                    del pk, pv
                else:
                    cache = fa.PagedKVCache.from_dense(k, v, block_size=page, lengths=lt, kv_format="fp8_block")
                kq, vq = fa.quantize_fp8_per_block(k, qb), fa.quantize_fp8_per_block(v, qb)
            elif qb == 1:
                cache = fa.PagedKVCache.from_dense(k, v, block_size=page, lengths=lt, kv_format="symmetric_token")
                kq, vq = fa.quantize_int8_symmetric_per_token(k), fa.quantize_int8_symmetric_per_token(v)
            else:
                if qb == page:
                    cache = fa.PagedKVCache.from_dense(k, v, block_size=page, lengths=lt, block_table_pattern=layout)
                else:
                    cache = paged_from_blocks(torch, fa, k, v, page, qb, lt)
                kq = fa.quantize_int8_per_block(k, qb)
                vq = fa.quantize_int8_per_block(v, qb)
            del k, v
            sets.append((q, cache, kq, vq, lt))
        ms = time_loop(torch, lambda i: fa.paged_quant_attention_triton(sets[i % n_sets][0], sets[i % n_sets][1]),
                       steps, warmup)
        _, st = fa.paged_quant_attention_triton(sets[0][0], sets[0][1], return_stats=True)
        row = {"shape": name, "format": fmt, "layout": layout, "batch": b, "heads": h, "seq_len": s, "head_dim": d, "page": page,
               "quant_block": qb, "q_dtype": qdt, "paged_us": round(ms * 1e3, 2), "paged_pct_of_peak": round(
                   100 * nbytes / (ms * 1e-3) / 1e9 / PEAK_GBPS, 1),
               "tiled_path": bool(st["tiled_path"]), "num_splits": st["num_splits"], "waves": st["num_warps"],
               "rotated_sets": n_sets, "rotated_bytes": n_sets * nbytes}
        fms = time_loop(torch, lambda i: fa.fused_dequant_attention_triton(
            sets[i % n_sets][0], sets[i % n_sets][2], sets[i % n_sets][3], lengths=sets[i % n_sets][4]), steps, warmup)
        row["fused_us"] = round(fms * 1e3, 2)
        row["paged_vs_fused"] = round(ms / fms, 3)
        out.append(row)
        print(json.dumps({"mode": "shapes", **row}), flush=True)
        del sets
        torch.cuda.empty_cache()
    return out


# (requests, draft-node counts, KV format of the prefix cache)
TREE_CASES = ((4, (1, 4, 8, 16, 32, 64), "affine_block"), (8, (16, 64), "affine_block"), (4, (16, 64), "fp8_block"))


def tree_bench(torch, fa, dev, steps: int, warmup: int) -> list[dict]:
    """tree_verify_attention over B4 and B8 H32 S4096 D128 paged prefixes (16-token pages, fp16
    q and drafts) for random draft trees of 1-64 nodes, `rotation_sets` input sets.  Algorithmic
    bytes read the shared prefix once per (request, head) plus the drafts, q, output and parents;
    ``vs_decode`` = time / the time of one single-query paged decode over the same prefix.  The
    tree topology is a host tensor, as a drafter produces it (checked, then copied through
    pinned memory inside the timed call)."""

    out = []
    g = torch.Generator(device=dev)
    g.manual_seed(13)
    gp = torch.Generator().manual_seed(17)
    for nb, node_counts, kv_format in TREE_CASES:
        prefix = algorithmic_bytes([S] * nb, H, D, PAGE, param_bytes=4 if kv_format == "fp8_block" else 6) \
            - 2 * nb * H * D * 2
        n_sets = rotation_sets(prefix)
        caches = []
        for _ in range(n_sets):
            k = torch.randn((nb, H, S, D), generator=g, device=dev, dtype=torch.float16)
            v = torch.randn((nb, H, S, D), generator=g, device=dev, dtype=torch.float16)
            caches.append(fa.PagedKVCache.from_dense(k, v, block_size=PAGE, kv_format=kv_format))
            del k, v
        q1 = [torch.randn((nb, H, D), generator=g, device=dev, dtype=torch.float16) for _ in range(n_sets)]
        dec_ms = time_loop(torch, lambda i: fa.paged_quant_attention_triton(q1[i % n_sets], caches[i % n_sets]),
                           steps, warmup)
        for n in node_counts:
            par = torch.full((nb, n), -1, dtype=torch.int64)
            for j in range(1, n):
                par[:, j] = torch.randint(-1, j, (nb,), generator=gp)
            ins = [tuple(torch.randn((nb, n, H, D), generator=g, device=dev, dtype=torch.float16) for _ in range(3))
                   for _ in range(n_sets)]
            ms = time_loop(torch, lambda i: fa.tree_verify_attention(ins[i % n_sets][0], caches[i % n_sets],
                                                                     ins[i % n_sets][1], ins[i % n_sets][2], par),
                           steps, warmup)
            _, st = fa.tree_verify_attention(ins[0][0], caches[0], ins[0][1], ins[0][2], par, return_stats=True)
            nbytes = prefix + 4 * nb * n * H * D * 2 + nb * n * 8
            row = {"workload": f"tree verify B{nb} H{H} S{S} D{D} {kv_format}, {n} draft nodes", "nodes": n,
                   "kv_format": kv_format,
                   "depth": st["tree_depth"], "us_per_call": round(ms * 1e3, 2), "algorithmic_bytes": nbytes,
                   "gbps": round(nbytes / (ms * 1e-3) / 1e9, 1),
                   "pct_of_peak": round(100 * nbytes / (ms * 1e-3) / 1e9 / PEAK_GBPS, 1),
                   "single_query_decode_us": round(dec_ms * 1e3, 2), "vs_decode": round(ms / dec_ms, 3),
                   "num_splits": st["num_splits"], "waves": st["num_warps"], "mfma_prefix": st["mfma_prefix"],
                   "nodes_per_workgroup": st["nodes_per_workgroup"], "rotated_sets": n_sets}
            out.append(row)
            print(json.dumps({"mode": "tree", **row}), flush=True)
            del ins
        del caches
        torch.cuda.empty_cache()
    return out


def load_traffic(config_key: str):
    if not PMC_SUMMARY.exists():
        return None
    try:
        d = json.loads(PMC_SUMMARY.read_text())
    except (OSError, ValueError):
        return None
    if d.get("config_key") != config_key:
        return None
    return d.get("hbm_bytes_per_launch")


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the decode path is sharded by "
              "(batch, head) rows with no cross-GPU exchange, so run one process per GPU instead.",
              file=sys.stderr)
        return 2
    import torch

    import flashspec_amd as fa
    from flashspec_amd import _lib

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    _lib.require()
    dev = torch.device("cuda", 0)
    if args.mode == "copy":
        return copy_calibration(torch, args.steps)
    if args.mode == "readbw":
        print(json.dumps({"mode": "readbw", **stream_read_ceiling(torch, dev, args.steps)}), flush=True)
        return 0
    if args.mode == "shapes":
        shapes_bench(torch, fa, dev, min(args.steps, 100), min(args.warmup, 10),
                     only={x for x in args.only.split(",") if x} or None)
        return 0
    if args.mode == "tree":
        tree_bench(torch, fa, dev, min(args.steps, 100), min(args.warmup, 10))
        return 0
    if args.mode == "serving":
        print(json.dumps({"mode": "serving", **serving_step_bench(torch, fa, dev, args.steps, args.warmup)}),
              flush=True)
        return 0
    sets = [make_inputs(torch, fa, dev, seed, args.layout) for seed in range(ROTATE)]
    torch.cuda.synchronize()
    lengths = [S] * B
    nbytes = algorithmic_bytes(lengths, H, D, PAGE)

    def paged_step(i):
        q, cache, _, _ = sets[i % ROTATE]
        return fa.paged_quant_attention_triton(q, cache)

    def paged_warm(i):
        q, cache, _, _ = sets[0]
        return fa.paged_quant_attention_triton(q, cache)

    def fused_step(i):
        q, _, kq, vq = sets[i % ROTATE]
        return fa.fused_dequant_attention_triton(q, kq, vq)

    _, stats = fa.paged_quant_attention_triton(sets[0][0], sets[0][1], return_stats=True)
    ms = time_loop(torch, paged_step, args.steps, args.warmup)
    if args.mode == "paged":
        print(json.dumps({"mode": "paged", "us_per_step": round(ms * 1e3, 2), "steps": args.steps,
                          "gbps": round(nbytes / (ms * 1e-3) / 1e9, 1)}), flush=True)
        return 0
    durs = kernel_durations_us(torch, paged_step, max(30, min(args.steps, 300)))
    kern_us = statistics.fmean(durs)
    warm_ms = time_loop(torch, paged_warm, args.steps, args.warmup)
    fused_ms = time_loop(torch, fused_step, args.steps, args.warmup)

    value = nbytes / (ms * 1e-3) / 1e9
    # At this shape one step is exactly one kernel launch (num_splits == 1: no merge
    # launch), so the timed-region events give the kernel's average launch duration; the
    # per-launch event pairs below add their own ~1 us and are reported for reference.
    single_launch = stats.get("num_splits", 1.0) == 1.0
    kernel_us = ms * 1e3 if single_launch else kern_us
    achieved = nbytes / (kernel_us * 1e-6) / 1e9
    config_key = f"paged_b{B}_h{H}_s{S}_d{D}_page{PAGE}_{args.layout}"
    result = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_s_per_timed_loop": SETTLE_S,
        "ms_per_step": round(ms, 5),
        "us_per_step": round(ms * 1e3, 2),
        "pct_of_peak": round(100.0 * value / PEAK_GBPS, 1),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": f"paged INT8 decode attention B{B} H{H} S{S} D{D}, {PAGE}-token pages, "
                        f"{args.layout} page layout, uniform lengths, {ROTATE} rotated input sets",
            "batch": B, "heads": H, "seq_len": S, "head_dim": D, "page_size": PAGE,
            "q_dtype": "float16", "kv_dtype": "int8 (per-page fp32 scale, int16 zero point)",
            "layout": args.layout, "rotated_input_sets": ROTATE, "parallelism": "single GPU",
            "num_splits": stats.get("num_splits"), "waves_per_workgroup": stats.get("num_warps"),
        },
        "algorithmic_bytes_per_step": nbytes,
        "warm_cache_us_per_step": round(warm_ms * 1e3, 2),
        "warm_cache_gbps": round(nbytes / (warm_ms * 1e-3) / 1e9, 1),
        "fused_contiguous_us_per_step": round(fused_ms * 1e3, 2),
        "paged_vs_fused_time_ratio": round(ms / fused_ms, 4),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_GBPS, 4),
            "traffic": load_traffic(config_key),
            "kernel": "decode_rows_kernel<128, __half, true, 0, 0> (paged_quant_attention)",
            "kernel_avg_us": round(kernel_us, 2),
            "kernel_avg_us_source": "timed-region HIP events / steps (one launch per step)" if single_launch
                                    else "per-launch HIP event pairs",
            "kernel_avg_us_event_pairs": round(kern_us, 2),
            "kernel_launches_timed": args.steps,
        },
        "device": torch.cuda.get_device_name(dev),
    }
    try:
        # contiguous rows: no block table, no lengths (269,352,960 bytes)
        result["c2_configured"] = c2_configured_bench(torch, fa, sets, args.steps, min(args.warmup, 300), fused_ms,
                                                      algorithmic_bytes(lengths, H, D, PAGE, idx_bytes=0) - 8 * B)
    except Exception as exc:  # reported, never hides the metric line
        result["c2_configured"] = {"error": f"{type(exc).__name__}: {exc}"}
    del sets
    torch.cuda.empty_cache()
    try:
        ceiling = stream_read_ceiling(torch, dev)
        result["stream_read"] = ceiling
        result["roofline"]["frac_of_stream_read"] = round(achieved / ceiling["GBps"], 4)
    except Exception as exc:  # reported, never hides the metric line
        result["stream_read"] = {"error": f"{type(exc).__name__}: {exc}"}
    torch.cuda.empty_cache()
    try:
        result["quantize"] = quantize_bench(torch, fa, dev)
    except Exception as exc:  # reported, never hides the metric line
        result["quantize"] = {"error": f"{type(exc).__name__}: {exc}"}
    torch.cuda.empty_cache()
    try:
        result["page_quantize"] = page_quantize_bench(torch, fa, dev)
    except Exception as exc:  # reported, never hides the metric line
        result["page_quantize"] = {"error": f"{type(exc).__name__}: {exc}"}
    torch.cuda.empty_cache()
    try:
        result["serving_step"] = serving_step_bench(torch, fa, dev, steps=min(args.steps, 50), warmup=5)
    except Exception as exc:  # reported, never hides the metric line
        result["serving_step"] = {"error": f"{type(exc).__name__}: {exc}"}
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(torch, fa, dev)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
