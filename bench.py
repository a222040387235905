"""Benchmark of the MI355X Sage attention forward (one GPU).

Workload: the headline shape B=1, H=30, N=4416, D=128 (1280x832 DiT image:
4160 image tokens + 256 text tokens), bf16 q/k/v ~ N(0,1) with a per-channel
K offset ~ N(0, 2), int8 QK (per-token scales) and fp8 P/V.  One "step" is one
full op call: sage_quantize_qkv (smoothing + quantization) followed by
sage_attn_fwd, with inputs resident in HBM.

Prints ONE JSON line.  ``value`` is TFLOP/s of the whole op on the
algorithmic count 4*B*H*N^2*D; ``roofline`` is the attention kernels (the
fused kernel plus the merge of the split tail items) against the dense 8-bit
MFMA peak; ``quantize`` reports the memory-bound kernels against HBM peak;
``cpu_baseline`` times the CPU oracle (the reference's algorithm restated in
PyTorch) on a bounded sample of the same workload on the host cores.

``--all-configs`` instead prints one JSON line per benchmark configuration
(the CPU plumbing case, 512x512, both 1280x832 variants, the packed
mixed-resolution batch with the reference tile mask and with exact document
ids, the k-tuple batch with key padding), each with its throughput, roofline
fraction and CPU baseline.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import torch

PEAK_8BIT_TFLOPS = 5000.0   # MI355X dense fp8 / int8 MFMA, TFLOP/s (TOP/s)
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E, GB/s

METRIC = "Sage attn fwd TFLOPS + ms/call at B=1,H=30,N=4416,D=128; % of fp8 MFMA peak"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # 1000 timed steps (about 0.28 s): shorter windows land in the clock and
    # power swings of the first second of load (measured on one box: 276-279
    # us per step over 1000-3000 steps, 283-294 over 20 steps after 5
    # warm-up, 306-312 over 100 steps after 150)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=150)
    # The GPU clock ramps during the first tens of milliseconds of work
    # (attention 318 us per call after 10 warm-up steps, 287 us after 150), so
    # before the counted warm-up the same op runs, untimed, for a fixed wall
    # time whatever --warmup says.
    ap.add_argument("--prewarm-seconds", type=float, default=0.3)
    ap.add_argument("--qk", default="int8", choices=["int8", "fp8"])
    ap.add_argument("--pv", default="fp8", choices=["fp8", "bf16"])
    ap.add_argument("--granularity", default="token", choices=["token", "block64"])
    ap.add_argument("--B", type=int, default=1)
    ap.add_argument("--H", type=int, default=30)
    ap.add_argument("--N", type=int, default=4416)
    ap.add_argument("--D", type=int, default=128)
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="approximate CPU time budget of the cpu_baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-sdpa", action="store_true",
                    help="--all-configs: skip the GPU scaled_dot_product_attention line of the unmasked cases")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="instead of the benchmark, run a plain device copy of MIB MiB "
                         "--steps times (scales the FETCH_SIZE / WRITE_SIZE counters)")
    ap.add_argument("--stream-calibration", action="store_true",
                    help="instead of the benchmark, time a 2:1 read/write stream at the quantization's "
                         "traffic and at 1 GiB, warm and cold")
    ap.add_argument("--phase-timing", action="store_true",
                    help="instead of the benchmark, run the headline op with the measurement build "
                         "(futudiffu_amd/build.py --phase-timing) and print the per-phase ticks of the "
                         "attention kernel's pipelined loop")
    ap.add_argument("--all-configs", action="store_true",
                    help="one JSON line per benchmark configuration instead of the headline line")
    ap.add_argument("--cases", default="",
                    help="comma-separated subset of the --all-configs cases")
    return ap.parse_args()


# Benchmark configurations: the CPU plumbing case, the 512x512 and 1280x832
# single-image shapes, the packed mixed-resolution batch (1280 + 1216 + 4416
# tokens) with the reference 128x64 tile mask and with exact document ids, and
# the k-tuple batch of four 1024x1024 samples with per-sample text padding.
CASES = {
    "plumbing_b1h4n256d64": dict(B=1, H=4, N=256, D=64, qk="int8", pv="bf16", gran="block64"),
    "dit512_b1h30n1280": dict(B=1, H=30, N=1280, D=128, qk="int8", pv="fp8", gran="token"),
    "dit1280x832_int8fp8": dict(B=1, H=30, N=4416, D=128, qk="int8", pv="fp8", gran="token"),
    "dit1280x832_fp8bf16": dict(B=1, H=30, N=4416, D=128, qk="fp8", pv="bf16", gran="token"),
    # the reference's fp8 LSE variant (fp8 QK, fp8 P.V: sage_attention.py:316-323)
    "dit1280x832_fp8fp8": dict(B=1, H=30, N=4416, D=128, qk="fp8", pv="fp8", gran="token"),
    # the production variant of futudiffu_ii::sage_attn_masked (int8 QK, bf16
    # P.V), unmasked and with the packed batch's reference tile mask
    "dit1280x832_int8bf16": dict(B=1, H=30, N=4416, D=128, qk="int8", pv="bf16", gran="token"),
    "packed_tilemask_int8bf16": dict(B=1, H=30, N=6912, D=128, qk="int8", pv="bf16", gran="token",
                                     segments=[1280, 1216, 4416], mask="tile"),
    "packed_tilemask": dict(B=1, H=30, N=6912, D=128, qk="int8", pv="fp8", gran="token",
                            segments=[1280, 1216, 4416], mask="tile"),
    "packed_docids": dict(B=1, H=30, N=6912, D=128, qk="int8", pv="fp8", gran="token",
                          segments=[1280, 1216, 4416], mask="doc"),
    "ktuple_b4n4352_keypad": dict(B=4, H=30, N=4352, D=128, qk="int8", pv="fp8", gran="token",
                                  mask="keypad", text=256),
    # the 1280x832 shape with the output stored as the out-projection's
    # [B, N, H*D] input, timed against [B, H, N, D] + the caller's transpose copy
    "dit1280x832_int8fp8_outproj": dict(B=1, H=30, N=4416, D=128, qk="int8", pv="fp8", gran="token",
                                        out="bnhd"),
    # the 1280x832 shape from the QKV projection output: the q/k/v producer
    # (RMSNorm + RoPE) inside the quantization, timed against the producer
    # writing bf16 q, k, v followed by the quantization
    "dit1280x832_int8fp8_from_qkv": dict(B=1, H=30, N=4416, D=128, qk="int8", pv="fp8", gran="token",
                                         producer=True),
    # the backward of the 1280x832 shape (int8 P recomputation, smoothing),
    # unmasked and with the packed batch's reference tile mask
    "dit1280x832_bwd_int8": dict(B=1, H=30, N=4416, D=128, qk="int8", pv="bf16", gran="token", bwd=True),
    "packed_tilemask_bwd_int8": dict(B=1, H=30, N=6912, D=128, qk="int8", pv="bf16", gran="token",
                                     segments=[1280, 1216, 4416], mask="tile", bwd=True),
    "packed_docids_bwd_int8": dict(B=1, H=30, N=6912, D=128, qk="int8", pv="bf16", gran="token",
                                   segments=[1280, 1216, 4416], mask="doc", bwd=True),
    "ktuple_b4n4352_keypad_bwd_int8": dict(B=4, H=30, N=4352, D=128, qk="int8", pv="bf16", gran="token",
                                           mask="keypad", text=256, bwd=True),
    # the producer's backward (RMSNorm + rotary gradients into the QKV
    # projection layout) at the 1280x832 shape
    "dit1280x832_producer_bwd": dict(B=1, H=30, N=4416, D=128, qk="int8", pv="bf16", gran="token",
                                     producer_bwd=True),
}
PEAK_MIXED_TFLOPS = 2.0 / (1.0 / PEAK_8BIT_TFLOPS + 1.0 / PEAK_BF16_TFLOPS)  # fp8 QK + bf16 PV


def quant_bytes(B, H, N, D, pv, gran):
    bh = B * H
    rd = 3 * bh * N * D * 2
    wr = 2 * bh * N * D + (bh * N * D if pv == "fp8" else 2 * bh * N * D)
    nsc = N if gran == "token" else (N + 63) // 64
    wr += 2 * bh * nsc * 4 + bh * D * 2
    if pv == "fp8":
        wr += bh * ((N + 63) // 64) * D * 4
    return rd + wr


def profiled_traffic(workload: str, kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE runs of this same workload (scaled by the copy calibration), or
    None when no profile of this workload is committed."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        "sage_fwd_int8qk_fp8pv_B1H30N4416D128_traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
    except OSError:
        return None
    if not workload.startswith(t["workload"]) or kernel not in t["kernels"]:
        return None
    k = t["kernels"][kernel]
    sc = t["counter_scale"]
    return round((k["fetch_kib"] * sc["FETCH_SIZE"] + k["write_kib"] * sc["WRITE_SIZE"]) * 1024)


def attn_bytes(B, H, N, D, pv, gran):
    """Algorithmic HBM bytes of one attention launch: codes, scales and V read once,
    output and LSE written once."""
    bh = B * H
    nsc = N if gran == "token" else (N + 63) // 64
    rd = 2 * bh * N * D + 2 * bh * nsc * 4 + bh * N * D * (1 if pv == "fp8" else 2)
    if pv == "fp8":
        rd += bh * ((N + 63) // 64) * D * 4
    return rd + bh * N * D * 2 + bh * N * 4


def cpu_baseline(args, flop_per_head):
    """Time the CPU oracle on whole heads of the same workload (bounded sample)."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import sage_oracle as O
    threads = torch.get_num_threads()
    q, k, v = O.make_inputs(1, 1, args.N, args.D, seed=123)
    t0 = time.perf_counter()
    O.sage_forward(q, k, v, None, args.qk, args.pv, args.granularity, True)
    one = time.perf_counter() - t0
    reps = max(1, min(8, int(args.cpu_seconds / max(one, 1e-3))))
    t0 = time.perf_counter()
    for _ in range(reps):
        O.sage_forward(q, k, v, None, args.qk, args.pv, args.granularity, True)
    per_head = (time.perf_counter() - t0) / reps
    sdpa_head = _median_seconds(lambda: torch.nn.functional.scaled_dot_product_attention(q, k, v))
    return {
        "value": round(flop_per_head / per_head / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"oracle (torch CPU emulation of the reference quantized attention) on "
                   f"{reps + 1} single-head runs B=1 H=1 N={args.N} D={args.D}; "
                   f"{per_head * 1e3:.1f} ms/head, full call extrapolated x{args.B * args.H}"),
        "ms_per_call_extrapolated": round(per_head * 1e3 * args.B * args.H, 3),
        "sdpa_bf16_cpu_ms_per_head": round(sdpa_head * 1e3, 3),
        "sdpa_sample": "torch SDPA on the same bf16 head, median of 3 runs after one warm-up run",
        "cpu_model": _cpu_model(),
        "os_cpu_count": os.cpu_count(),
    }


def _median_seconds(fn, runs=3):
    """Median wall time of ``runs`` calls of ``fn`` after one untimed call."""
    fn()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return sorted(times)[len(times) // 2]


class TimingEvent:
    """A HIP event on torch's current stream (the stream the library launches
    on), created with hipEventDisableSystemFence: recording it skips the
    system-scope fence, a cache write-back and invalidation that otherwise
    stalls the next kernel by several microseconds (measured: 308 -> 289 us
    per headline step with a pair of events around each op).  The events are
    used only for timing, as that flag requires; the host synchronizes the
    device before reading them."""

    _hip = None
    _DISABLE_SYSTEM_FENCE = 0x20000000

    @classmethod
    def _runtime(cls):
        if cls._hip is None:
            import ctypes
            path = None
            with open("/proc/self/maps") as f:  # the HIP runtime torch loaded
                for line in f:
                    if "libamdhip64.so" in line:
                        path = line.split()[-1]
                        break
            if path is None:
                raise RuntimeError("the HIP runtime is not loaded")
            hip = ctypes.CDLL(path)
            hip.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
            hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
            hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
            hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
            cls._hip = hip
        return cls._hip

    def __init__(self):
        import ctypes
        hip = self._runtime()
        self._ev = ctypes.c_void_p()
        if hip.hipEventCreateWithFlags(ctypes.byref(self._ev), self._DISABLE_SYSTEM_FENCE) != 0:
            raise RuntimeError("hipEventCreateWithFlags failed")

    def record(self):
        if self._hip.hipEventRecord(self._ev, torch.cuda.current_stream().cuda_stream) != 0:
            raise RuntimeError("hipEventRecord failed")

    def elapsed_time(self, end) -> float:
        import ctypes
        ms = ctypes.c_float()
        if self._hip.hipEventElapsedTime(ctypes.byref(ms), self._ev, end._ev) != 0:
            raise RuntimeError("hipEventElapsedTime failed (synchronize first)")
        return ms.value

    def __del__(self):
        if self._hip is not None and getattr(self, "_ev", None):
            self._hip.hipEventDestroy(self._ev)


def prewarm(step, seconds):
    """Run ``step`` untimed until ``seconds`` of wall time have passed (the
    device synchronized), so the counted warm-up starts at steady clocks.
    The device is synchronized only every 64 steps: an idle gap after every
    few steps lets the clocks drop again."""
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    n = 0
    while True:
        for _ in range(64):
            step()
        n += 64
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= seconds:
            return {"seconds": round(time.perf_counter() - t0, 4), "steps": n}


def sdpa_gpu(qd, kd, vd, sm, args):
    """torch's scaled_dot_product_attention on the same bf16 q, k, v on the
    GPU, the comparison the reference publishes for its Sage op
    (bench/bench_attention.py:57-58): median over --steps calls between HIP
    events, after the same pre-warm and warm-up.  Only the fused backends
    (flash, then memory-efficient) are allowed: the unfused math path forms
    the N x N scores with batched bf16 products of a transposed operand.
    Context for the comparison, not part of the measured op."""
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel
    B, H, N, D = qd.shape
    flop = 4.0 * B * H * N * N * D
    for name, backend in (("flash", SDPBackend.FLASH_ATTENTION), ("efficient", SDPBackend.EFFICIENT_ATTENTION)):
        try:
            with sdpa_kernel([backend]):
                def call():
                    F.scaled_dot_product_attention(qd, kd, vd, scale=sm)
                call()
                torch.cuda.synchronize()
                prewarm(call, args.prewarm_seconds)
                for _ in range(args.warmup):
                    call()
                evs = [(TimingEvent(), TimingEvent()) for _ in range(args.steps)]
                for e in evs:
                    e[0].record()
                    call()
                    e[1].record()
                torch.cuda.synchronize()
        except RuntimeError as err:
            last = f"{name}: {str(err).splitlines()[0][:160]}"
            continue
        ms = sorted(e[0].elapsed_time(e[1]) for e in evs)[len(evs) // 2]
        tf = flop / (ms * 1e-3) / 1e12
        return {"backend": name, "dtype": "bf16", "ms": round(ms, 5), "tflops": round(tf, 2),
                "frac_of_bf16_peak": round(tf / PEAK_BF16_TFLOPS, 4)}
    return {"unavailable": last}


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def copy_calibration(args):
    """Plain copy of a known size: the reference point for HBM byte counters."""
    nbytes = args.copy_calibration << 20
    src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(args.steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes_read": nbytes, "copy_calibration_bytes_written": nbytes,
                      "launches": args.steps}), flush=True)


def stream_rate(total_bytes: int, cold: bool, reps: int = 9) -> float:
    """GB/s of a 2:1 read/write stream moving ``total_bytes`` per launch:
    torch.add of two bf16 tensors into a third (reads two, writes one, the
    quantization's ratio).  warm: the same buffers back to back, resident in
    the 256 MB Infinity Cache when they fit.  cold: a 1 GiB fill runs before
    each timed launch.  Median over ``reps`` launches, timed with HIP events."""
    n = total_bytes // 6
    a = torch.randn(n, device="cuda:0").bfloat16()
    b = torch.randn(n, device="cuda:0").bfloat16()
    c = torch.empty_like(a)
    flush = torch.empty(1 << 30, dtype=torch.uint8, device="cuda:0") if cold else None
    for _ in range(3):
        torch.add(a, b, out=c)
    times = []
    for _ in range(reps):
        if cold:
            flush.fill_(1)
        e0, e1 = TimingEvent(), TimingEvent()
        e0.record()
        torch.add(a, b, out=c)
        e1.record()
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1))
    ms = sorted(times)[len(times) // 2]
    return 6 * n / (ms * 1e-3) / 1e9


def stream_calibration(args):
    """The 2:1 stream at the quantization's traffic of the headline shape and
    at 1 GiB, warm and after a 1 GiB fill."""
    qb = quant_bytes(args.B, args.H, args.N, args.D, args.pv, args.granularity)
    out = {"stream": "torch.add of two bf16 tensors into a third (2 bytes read per byte written)",
           "quantize_traffic_bytes": qb}
    for label, nbytes in (("quantize_traffic", qb), ("1GiB", 1 << 30)):
        for cold in (False, True):
            out[f"{label}_{'cold' if cold else 'warm'}_GBs"] = round(stream_rate(nbytes, cold), 1)
    print(json.dumps(out), flush=True)


def _case_inputs(c, dev, seed=0):
    """Seeded q/k/v of a case (K with a per-channel N(0, 2) offset), its masks,
    and its algorithmic FLOP count (visible query-key pairs x 4D)."""
    B, H, N, D = c["B"], c["H"], c["N"], c["D"]
    g = torch.Generator(device="cpu").manual_seed(seed)
    q = torch.randn(B, H, N, D, generator=g).bfloat16()
    k = (torch.randn(B, H, N, D, generator=g) + 2.0 * torch.randn(B, H, 1, D, generator=g)).bfloat16()
    v = torch.randn(B, H, N, D, generator=g).bfloat16()
    mask = c.get("mask")
    block_mask = doc = None
    flop = 4.0 * B * H * N * N * D
    extra = {}
    if mask in ("tile", "doc"):
        from futudiffu_amd import block_mask as BM
        segs = c["segments"]
        flop = 4.0 * B * H * D * sum(x * x for x in segs)
        extra["flop_dense"] = 4.0 * B * H * N * N * D
        if mask == "tile":
            block_mask = BM.build_block_mask(segs, N, device="cpu")
            extra["tile_skip_efficiency"] = round(float(block_mask.float().mean()), 4)
            extra["active_tiles"] = int(block_mask.sum())
            extra["total_tiles"] = int(block_mask.numel())
        else:
            doc = BM.build_doc_ids(segs, N, device="cpu", batch=B)
    elif mask == "keypad":
        # text first: sample b keeps L_b ~ U[32, 256] of its 256 text slots, the
        # rest of the text slots are padding keys; all image tokens are valid
        gl = torch.Generator(device="cpu").manual_seed(seed + 1)
        lens = torch.randint(32, c["text"] + 1, (B,), generator=gl)
        valid = torch.ones(B, N, dtype=torch.bool)
        for b in range(B):
            valid[b, int(lens[b]):c["text"]] = False
        doc = torch.where(valid, 0, -1).to(torch.int32)
        nvalid = valid.sum(dim=1).double()
        # every query (padded ones included) attends the valid keys of its sample
        flop = float(4.0 * H * D * N * nvalid.sum())
        extra["flop_dense"] = 4.0 * B * H * N * N * D
        extra["text_lengths"] = [int(x) for x in lens]
    return q, k, v, block_mask, doc, flop, extra


def _cpu_case(c, q, k, v, block_mask, doc, flop, budget_s):
    """CPU oracle and CPU SDPA on one head of batch 0 of the case (bounded)."""
    from oracle import sage_oracle as O
    N = c["N"]
    q1, k1, v1 = q[:1, :1], k[:1, :1], v[:1, :1]
    d1 = None if doc is None else doc[:1]
    t0 = time.perf_counter()
    O.sage_forward(q1, k1, v1, None, c["qk"], c["pv"], c["gran"], True, block_mask, d1)
    per_head = time.perf_counter() - t0
    reps = 0
    if per_head < budget_s / 2:
        reps = max(1, min(4, int(budget_s / per_head) - 1))
        t0 = time.perf_counter()
        for _ in range(reps):
            O.sage_forward(q1, k1, v1, None, c["qk"], c["pv"], c["gran"], True, block_mask, d1)
        per_head = (time.perf_counter() - t0) / reps
    heads = c["B"] * c["H"]
    vis = None
    if block_mask is not None:
        vis = O.tile_mask_visibility(block_mask, 1, N)
    if d1 is not None:
        dv = O.doc_visibility(d1.to(torch.int64))
        vis = dv if vis is None else vis & dv
    am = None if vis is None else vis[:, None]
    sdpa = _median_seconds(lambda: torch.nn.functional.scaled_dot_product_attention(q1, k1, v1, attn_mask=am))
    return {
        "value": round(flop / heads / per_head / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"oracle (torch CPU emulation of the reference quantized attention) on {reps + 1} run(s) "
                   f"of one head (batch 0, head 0) of this case; {per_head * 1e3:.1f} ms/head, "
                   f"throughput on that head's share of the FLOPs"),
        "sdpa_bf16_cpu_ms_per_head": round(sdpa * 1e3, 3),
        "sdpa_sample": "torch SDPA on the same bf16 head and mask, median of 3 runs after one warm-up run",
        "cpu_model": _cpu_model(),
    }


def backward_case(args, name, c):
    """Time the backward (quantization + operand images + D pre-pass + dK/dV +
    dQ) on the forward's output.  Algorithmic FLOP = 10 * (visible pairs) * D:
    the S recomputation (int8 / fp8), dP, dV, dK and dQ (2 each, the last four
    bf16); the MFMA bound prices the first at the 8-bit peak and the rest at
    the bf16 peak."""
    from futudiffu_amd import sage_attention as SA
    dev = torch.device("cuda:0")
    B, H, N, D = c["B"], c["H"], c["N"], c["D"]
    q, k, v, bm, doc, flop_fwd, extra = _case_inputs(c, dev)
    pairs_d = flop_fwd / 4.0
    flop = 10.0 * pairs_d
    bound_s = 2.0 * pairs_d / (PEAK_8BIT_TFLOPS * 1e12) + 8.0 * pairs_d / (PEAK_BF16_TFLOPS * 1e12)
    sm = 1.0 / math.sqrt(D)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    bmd = None if bm is None else bm.to(dev)
    docd = None if doc is None else doc.to(dev)
    g = torch.Generator(device="cpu").manual_seed(7)
    dout = torch.randn(B, H, N, D, generator=g).bfloat16()
    dod = dout.to(dev)
    out, lse = SA.sage_forward(qd, kd, vd, sm, block_mask=bmd, doc_ids=docd, qk=c["qk"], pv=c["pv"], smooth_k=True)

    def step():
        return SA.sage_backward(qd, kd, vd, out, lse, dod, sm, block_mask=bmd, doc_ids=docd, qk=c["qk"],
                                smooth_k=True)

    prewarm(step, args.prewarm_seconds)
    for _ in range(max(args.warmup // 4, 10)):
        step()
    torch.cuda.synchronize()
    e0, e1 = TimingEvent(), TimingEvent()
    steps = max(args.steps // 4, 5)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    tf = flop / (ms * 1e-3) / 1e12
    line = {
        "case": name,
        "config": {k2: v2 for k2, v2 in c.items()},
        "bwd_ms": round(ms, 5),
        "bwd_tflops": round(tf, 2),
        "flop": flop,
        "roofline": {"bound": "mfma", "unit": "ms", "bound_ms": round(bound_s * 1e3, 5),
                     "frac": round(bound_s * 1e3 / ms, 4),
                     "peaks": f"S at {PEAK_8BIT_TFLOPS} TFLOP/s, dP/dV/dK/dQ at {PEAK_BF16_TFLOPS} TFLOP/s"},
    }
    line.update({k2: v2 for k2, v2 in extra.items() if k2 != "flop_dense"})
    if not args.no_cpu_baseline:
        from oracle import sage_oracle as O
        q1, k1, v1, d1 = q[:1, :1], k[:1, :1], v[:1, :1], dout[:1, :1]
        bm1 = None if bm is None else bm
        doc1 = None if doc is None else doc[:1]
        o1, l1, _ = O.sage_forward(q1, k1, v1, sm, c["qk"], "bf16", "token", True, bm1, doc1)
        t0 = time.perf_counter()
        O.sage_backward(q1, k1, v1, o1, l1, d1, sm, qk=c["qk"], smooth=True, block_mask=bm1, doc_ids=doc1,
                        head_chunk=1)
        per_head = time.perf_counter() - t0
        line["cpu_baseline"] = {
            "value": round(flop / (B * H) / per_head / 1e12, 6), "unit": "TFLOP/s",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"oracle backward (torch CPU restatement) of one head (batch 0, head 0): "
                      f"{per_head * 1e3:.1f} ms/head, throughput on that head's share of the FLOPs",
            "cpu_model": _cpu_model()}
    print(json.dumps(line), flush=True)


def producer_backward_case(args, name, c):
    """Time the producer's backward (``qkv_postprocess_backward``).
    Algorithmic bytes: the q and k rows of the projection output and the
    three incoming gradients read (5 * B*N*H*D bf16), the three rotation
    entries per channel pair and token read once (12 * B*N*D/2), dqkv written
    (3 * B*N*H*D bf16)."""
    from futudiffu_amd import sage_attention as SA
    dev = torch.device("cuda:0")
    B, H, N, D = c["B"], c["H"], c["N"], c["D"]
    g = torch.Generator(device="cpu").manual_seed(3)
    qkv = torch.randn(B, N, 3 * H * D, generator=g).bfloat16()
    nw = 1.0 + 0.1 * torch.randn(2, D, generator=g)
    ang = torch.rand(B, N, 1, D // 2, generator=g) * 6.283
    cs, sn = torch.cos(ang), torch.sin(ang)
    freqs = torch.stack([torch.stack([cs, -sn], -1), torch.stack([sn, cs], -1)], -2)
    grads = [torch.randn(B, H, N, D, generator=g).bfloat16() for _ in range(3)]
    dv = [t.to(dev) for t in (qkv, nw[0], nw[1], freqs, *grads)]

    def step():
        return SA.qkv_postprocess_backward(*dv, H, D, 1e-5)

    prewarm(step, args.prewarm_seconds)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = TimingEvent(), TimingEvent()
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    nbytes = 5 * B * N * H * D * 2 + 12 * B * N * (D // 2) + 3 * B * N * H * D * 2
    gbs = nbytes / (ms * 1e-3) / 1e9
    line = {
        "case": name,
        "config": {k2: v2 for k2, v2 in c.items()},
        "producer_bwd_ms": round(ms, 5),
        "bytes": nbytes,
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_HBM_GBS, 4)},
    }
    if not args.no_cpu_baseline:
        from oracle import sage_oracle as O
        t0 = time.perf_counter()
        O.qkv_postprocess_backward(qkv, nw[0], nw[1], freqs, *grads, H, D, 1e-5)
        sec = time.perf_counter() - t0
        line["cpu_baseline"] = {
            "value": round(nbytes / sec / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(),
            "kind": "port", "sample": f"oracle producer backward (torch CPU, fp64) on the whole case: "
                                      f"{sec * 1e3:.1f} ms", "cpu_model": _cpu_model()}
    print(json.dumps(line), flush=True)


def all_configs(args):
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from futudiffu_amd import sage_attention as SA
    dev = torch.device("cuda:0")
    names = [x for x in args.cases.split(",") if x] or list(CASES)
    for name in names:
        c = CASES[name]
        B, H, N, D = c["B"], c["H"], c["N"], c["D"]
        print(f"# case {name}", file=sys.stderr, flush=True)
        if c.get("bwd"):
            backward_case(args, name, c)
            continue
        if c.get("producer_bwd"):
            producer_backward_case(args, name, c)
            continue
        q, k, v, bm, doc, flop, extra = _case_inputs(c, dev)
        qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
        bmd = None if bm is None else bm.to(dev)
        docd = None if doc is None else doc.to(dev)
        sm = 1.0 / math.sqrt(D)
        layout = c.get("out", "bhnd")
        if c.get("producer"):
            g = torch.Generator(device="cpu").manual_seed(1)
            qkv = torch.randn(B, N, 3 * H * D, generator=g).bfloat16().to(dev)
            nw = (1.0 + 0.1 * torch.randn(2, D, generator=g)).to(dev)
            ang = torch.rand(B, N, 1, D // 2, generator=g) * 6.283
            cs, sn = torch.cos(ang), torch.sin(ang)
            freqs = torch.stack([torch.stack([cs, -sn], -1), torch.stack([sn, cs], -1)], -2).to(dev)

        def quantize(fused=True):
            if not c.get("producer"):
                return SA.quantize_qkv(qd, kd, vd, sm, qk=c["qk"], pv=c["pv"], granularity=c["gran"])
            if fused:
                return SA.quantize_from_qkv(qkv, nw[0], nw[1], freqs, H, D, 1e-5, sm, qk=c["qk"], pv=c["pv"],
                                            granularity=c["gran"])
            qq, kk, vv = SA.qkv_postprocess(qkv, nw[0], nw[1], freqs, H, D, 1e-5)
            return SA.quantize_qkv(qq, kk, vv, sm, qk=c["qk"], pv=c["pv"], granularity=c["gran"])

        def step(ev=None, out_layout=layout, merge_heads=False, fused=True):
            if ev is not None:
                ev[0].record()
            qz = quantize(fused)
            if ev is not None:
                ev[1].record()
            out, _ = SA.attn_from_quantized(qz, B, H, block_mask=bmd, doc_ids=docd, out_layout=out_layout)
            if merge_heads:  # the caller's copy into the out-projection layout (transformer.py:471)
                out.transpose(1, 2).reshape(B, -1, H * D)
            if ev is not None:
                ev[2].record()

        def timed(**kw):
            prewarm(lambda: step(**kw), args.prewarm_seconds)
            for _ in range(args.warmup):
                step(**kw)
            torch.cuda.synchronize()
            evs = [[TimingEvent() for _ in range(3)] for _ in range(args.steps)]
            for i in range(args.steps):
                step(evs[i], **kw)
            torch.cuda.synchronize()
            return (sum(e[1].elapsed_time(e[2]) for e in evs) / args.steps,
                    sum(e[0].elapsed_time(e[1]) for e in evs) / args.steps)

        a_ms, q_ms = timed()
        if c.get("producer"):
            _, sep_q_ms = timed(fused=False)
            extra["from_qkv"] = {"producer_in_quantize_ms": round(q_ms, 5),
                                 "producer_then_quantize_ms": round(sep_q_ms, 5),
                                 "saved_ms": round(sep_q_ms - q_ms, 5),
                                 "note": "quantize columns include the producer (RMSNorm + RoPE) in both forms"}
        if layout == "bnhd":
            sep_ms, _ = timed(out_layout="bhnd", merge_heads=True)
            extra["outproj_input"] = {"fused_bnhd_store_ms": round(a_ms, 5),
                                      "bhnd_store_plus_transpose_copy_ms": round(sep_ms, 5),
                                      "saved_ms": round(sep_ms - a_ms, 5)}
        tf = flop / (a_ms * 1e-3) / 1e12
        qb = quant_bytes(B, H, N, D, c["pv"], c["gran"])
        line = {
            "case": name,
            "config": {k2: v2 for k2, v2 in c.items()},
            "attn_ms": round(a_ms, 5),
            "attn_tflops": round(tf, 2),
            "flop": flop,
            "roofline": {"bound": "mfma", "peak": PEAK_8BIT_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tf / PEAK_8BIT_TFLOPS, 4)},
            "quantize": {"ms": round(q_ms, 5), "GB/s": round(qb / (q_ms * 1e-3) / 1e9, 1),
                         "frac_of_hbm_peak": round(qb / (q_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)},
            "op_ms": round(a_ms + q_ms, 5),
        }
        if c["pv"] == "bf16" and c["qk"] == "fp8":
            line["roofline"]["frac_of_mixed_fp8_bf16_peak"] = round(tf / PEAK_MIXED_TFLOPS, 4)
        line.update(extra)
        if not args.no_sdpa and bm is None and doc is None and not c.get("producer") and layout == "bhnd":
            s = sdpa_gpu(qd, kd, vd, sm, args)
            if "ms" in s:
                s["sage_op_speedup"] = round(s["ms"] / (a_ms + q_ms), 3)
            line["sdpa_gpu_same_inputs"] = s
        if not args.no_cpu_baseline:
            line["cpu_baseline"] = _cpu_case(c, q, k, v, bm, doc, flop, args.cpu_seconds)
        print(json.dumps(line), flush=True)


PHASE_NAMES = ["loop overhead", "stage loads issued + pending P.V + score conversion", "next QK^T issue",
               "row max + frame decision", "exp + row sums + P packing", "stage-load wait + barrier"]


def phase_timing(args):
    """Per-phase s_memtime ticks of the attention kernel's pipelined loop
    (one iteration = one 32-row x 64-key tile of one wave), summed over every
    live wave of --steps headline calls, from the measurement library.  The
    scheduling fences at the phase boundaries keep each phase's instructions
    inside it, so the instrumented kernel runs slower than the product one;
    the split shows where a wave's time goes."""
    import ctypes
    root = os.path.dirname(os.path.abspath(__file__))
    path = os.path.join(root, "futudiffu_amd", "libsage_mi355x_phase.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built: python futudiffu_amd/build.py --phase-timing")
    os.environ["SAGE_MI355X_LIB"] = path
    sys.path.insert(0, root)
    from futudiffu_amd import _lib
    from futudiffu_amd import sage_attention as SA
    lib = _lib.load()
    lib.sage_phase_read.restype = ctypes.c_int
    lib.sage_phase_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    B, H, N, D = args.B, args.H, args.N, args.D
    dev = torch.device("cuda:0")
    g = torch.Generator(device="cpu").manual_seed(0)
    q = torch.randn(B, H, N, D, generator=g).bfloat16().to(dev)
    k = (torch.randn(B, H, N, D, generator=g) + 2.0 * torch.randn(B, H, 1, D, generator=g)).bfloat16().to(dev)
    v = torch.randn(B, H, N, D, generator=g).bfloat16().to(dev)
    qz = SA.quantize_qkv(q, k, v, 1.0 / math.sqrt(D), qk=args.qk, pv=args.pv, granularity=args.granularity)
    prewarm(lambda: SA.attn_from_quantized(qz, B, H), args.prewarm_seconds)
    torch.cuda.synchronize()
    if lib.sage_phase_read(None, 0, 1) != 0:
        raise RuntimeError("sage_phase_read failed")
    evs = [(TimingEvent(), TimingEvent()) for _ in range(args.steps)]
    for e in evs:
        e[0].record()
        SA.attn_from_quantized(qz, B, H)
        e[1].record()
    torch.cuda.synchronize()
    slots = 32768
    buf = (ctypes.c_ulonglong * (slots * 8))()
    if lib.sage_phase_read(buf, slots * 8, 1) != 0:
        raise RuntimeError("sage_phase_read failed")
    rows = [buf[i * 8:(i + 1) * 8] for i in range(slots)]
    rows = [r for r in rows if r[6] > 0]
    iters = sum(r[6] for r in rows)
    tot = [sum(r[k] for r in rows) for k in range(6)]
    loop_ticks = sum(r[7] for r in rows)
    per = [t / iters for t in tot]
    ms = sorted(e[0].elapsed_time(e[1]) for e in evs)[len(evs) // 2]
    print(json.dumps({
        "phase_timing": f"attn_fwd_kernel {args.qk}-QK {args.pv}-PV B={B} H={H} N={N} D={D}, {args.steps} calls",
        "instrumented_kernel_ms_median": round(ms, 5),
        "waves_timed": len(rows), "iterations": iters,
        "ticks_per_iteration": round(sum(per), 1),
        "phases": [{"phase": PHASE_NAMES[k], "ticks_per_iteration": round(per[k], 1),
                    "share": round(per[k] / sum(per), 4)} for k in range(6)],
        "loop_ticks_outside_timed_iterations_share": round(1 - sum(tot) / loop_ticks, 4),
        "unit": "s_memtime ticks per wave per 32x64 tile",
    }), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(the forward shards by head with no exchange between GPUs)", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    if args.copy_calibration:
        copy_calibration(args)
        return
    if args.stream_calibration:
        stream_calibration(args)
        return
    if args.phase_timing:
        phase_timing(args)
        return
    if args.all_configs:
        all_configs(args)
        return
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from futudiffu_amd import sage_attention as SA

    B, H, N, D = args.B, args.H, args.N, args.D
    dev = torch.device("cuda:0")
    g = torch.Generator(device="cpu").manual_seed(0)
    q = torch.randn(B, H, N, D, generator=g).bfloat16().to(dev)
    k = (torch.randn(B, H, N, D, generator=g) + 2.0 * torch.randn(B, H, 1, D, generator=g)).bfloat16().to(dev)
    v = torch.randn(B, H, N, D, generator=g).bfloat16().to(dev)
    sm = 1.0 / math.sqrt(D)
    flop = 4.0 * B * H * N * N * D

    def step(ev=None):
        if ev is not None:
            ev[0].record()
        qz = SA.quantize_qkv(q, k, v, sm, qk=args.qk, pv=args.pv, granularity=args.granularity)
        if ev is not None:
            ev[1].record()
        out = SA.attn_from_quantized(qz, B, H)
        if ev is not None:
            ev[2].record()
        return out

    warm = prewarm(step, args.prewarm_seconds)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    evs = [[TimingEvent() for _ in range(3)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(evs[i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    qms = sorted(e[0].elapsed_time(e[1]) for e in evs)
    ams = sorted(e[1].elapsed_time(e[2]) for e in evs)
    ms_per_step = wall * 1e3 / args.steps
    q_stream = stream_rate(quant_bytes(B, H, N, D, args.pv, args.granularity), cold=False)
    q_avg = sum(qms) / len(qms)
    a_avg = sum(ams) / len(ams)

    workload = (f"sage_attn_fwd B={B} H={H} N={N} D={D} {args.qk}-QK {args.pv}-PV "
                f"{args.granularity} scales, no mask (quantize + fused attention)")
    attn_tflops = flop / (a_avg * 1e-3) / 1e12
    peak = PEAK_8BIT_TFLOPS
    qbytes = quant_bytes(B, H, N, D, args.pv, args.granularity)
    q_gbs = qbytes / (q_avg * 1e-3) / 1e9

    res = {
        "metric": METRIC,
        "value": round(flop / (ms_per_step * 1e-3) / 1e12, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": f"{args.qk}-qk/{args.pv}-pv",
        "data": "synthetic: q,k,v ~ N(0,1) bf16, K += N(0,2) per channel, seed 0",
        "config": {
            "workload": workload,
            "B": B, "H": H, "N": N, "D": D, "qk": args.qk, "pv": args.pv,
            "granularity": args.granularity, "parallelism": "single GPU",
        },
        "pct_of_fp8_peak": round(100.0 * flop / (ms_per_step * 1e-3) / 1e12 / PEAK_8BIT_TFLOPS, 2),
        "prewarm": {**warm, "note": "untimed run of the same op before the counted warm-up (clock ramp)"},
        "roofline": {
            "bound": "mfma",
            "kernel": "attn_fwd_kernel (split tail items merged inside it)",
            "achieved": round(attn_tflops, 3),
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": round(attn_tflops / peak, 4),
            "traffic": profiled_traffic(workload, "attn_fwd_kernel"),
            "traffic_unit": "bytes per launch (rocprofv3 FETCH_SIZE x2.0 + WRITE_SIZE x1.0)",
            "algorithmic_bytes": attn_bytes(B, H, N, D, args.pv, args.granularity),
            "avg_kernel_ms": round(a_avg, 5),
            "median_kernel_ms": round(ams[len(ams) // 2], 5),
            "flop_per_launch": flop,
        },
        "quantize": {
            "bound": "hbm",
            "kernel": "quantize_one_kernel (K column sums, then the Q, V and K blocks)",
            "achieved": round(q_gbs, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(q_gbs / PEAK_HBM_GBS, 4),
            "algorithmic_bytes": qbytes,
            "traffic": profiled_traffic(workload, "quantize_one_kernel"),
            "traffic_unit": "bytes per launch (rocprofv3 FETCH_SIZE x2.0 + WRITE_SIZE x1.0; K is read twice)",
            "avg_ms": round(q_avg, 5),
            # the same traffic as a plain 2:1 stream, measured here after the timed steps
            "stream_2to1_GBs": round(q_stream, 1),
            "frac_of_stream": round(q_gbs / q_stream, 4),
        },
    }
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(args, flop / (B * H))
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
