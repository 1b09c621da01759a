"""OpWorks-on-MI355X benchmark driver (one JSON line on stdout).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--no-cpu]

A "step" is one pass of the hot path over one batch of synthetic input already
resident in HBM. Timing uses HIP events recorded on the stream the kernels are
launched on, bracketed by a device synchronize on both sides; the average
launch duration is K events apart divided by K. Working sets smaller than
512 MiB are rotated over several buffer sets so the 256 MB Infinity Cache
cannot serve them.

`value` is the headline workload's throughput; every measured workload also
appears under `components` with its own roofline. `cpu_baseline` times the CPU
oracle (the restatement of the reference kernels) on a bounded sample on this
host: the headline's at the top level, every other workload's in its component.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

import opworks_amd as ow  # noqa: E402

HBM_PEAK_GBS = 8000.0
FP32_PEAK_TFLOPS = 157.3
BF16_PEAK_TFLOPS = 2500.0
SEED = 1234
METRIC = json.loads((ROOT / "BASELINE.json").read_text())["metric"]


def cpu_threads() -> int:
    """Threads the CPU baseline uses: every CPU this process may run on, at most 16 (the GPU pool's CPU
    share per GPU, whatever nproc reports there)."""
    try:
        available = len(os.sched_getaffinity(0))
    except AttributeError:
        available = os.cpu_count() or 1
    return max(1, min(16, available))


class Timer:
    """K launches (more for short ops: at least MIN_TIMED_MS of them, at most MAX_LAUNCHES) between two
    events on `stream`, synchronized on both sides; returns the average per launch.

    A launch from Python (ctypes + the HIP runtime) takes several microseconds of host time, longer
    than a softmax step runs on the GPU. So before the first event an untimed filler (a copy over
    512 MiB, ~0.17 ms per pass, enough passes to cover the host's enqueue time for the K steps) is
    queued on the same stream. The K steps then wait in the queue while the filler runs, and the
    events measure the GPU's back-to-back execution of the K steps, not the host's launch rate.

    The engine clock of an idle MI355X ramps up over roughly 100 ms of load, so an op whose step
    keeps the GPU busy for longer than a host launch takes (>= PREWARM_MIN_MS) first runs back to
    back, untimed, for PREWARM_S of wall time: its K steps are then timed at the clocks of a busy
    GPU (the steady state a serving loop sees). Shorter ops are not pre-run: launched from Python
    they would leave the GPU idle between steps, which is not a steady state of theirs (softmax
    measured slower after such a run, not faster)."""

    _filler = None
    FILL_N = 1 << 27  # floats per filler buffer (512 MiB)
    PREWARM_S = 0.25
    PREWARM_MIN_MS = 0.05
    MIN_TIMED_MS = 2.0
    MAX_LAUNCHES = 1024

    def __init__(self, stream):
        self.stream = stream
        self.t0, self.t1 = ow.Event(), ow.Event()

    def _fill(self, steps: int) -> None:
        if Timer._filler is None:
            Timer._filler = (ow.DeviceBuffer.empty(self.FILL_N), ow.DeviceBuffer.empty(self.FILL_N))
        src, dst = Timer._filler
        for _ in range(1 + steps // 4):  # ~0.17 ms of GPU time per 4 steps of host enqueue
            ow.ops.copy(src, dst, self.FILL_N, stream=self.stream)

    def _prewarm(self, fn) -> float:
        """Returns one launch's duration in ms (the second launch: the first also loads the code object)."""
        fn(0)
        self.t0.record(self.stream)
        fn(1)
        self.t1.record(self.stream)
        self.t1.synchronize()
        est = self.t0.elapsed_ms(self.t1)
        if est < self.PREWARM_MIN_MS:
            return est
        t0, i = time.perf_counter(), 2
        while time.perf_counter() - t0 < self.PREWARM_S:
            for _ in range(8):  # bounded queue: at most 8 steps ahead of the host
                fn(i)
                i += 1
            ow.check(ow.lib().opw_device_synchronize())
        return est

    def run(self, fn, steps: int, warmup: int) -> float:
        est = self._prewarm(fn)
        # Short ops are timed over at least MIN_TIMED_MS of back-to-back launches (K if that is more):
        # a 20-launch window of a 6 us kernel varied by 15% between runs.
        timed = max(steps, min(self.MAX_LAUNCHES, int(self.MIN_TIMED_MS / max(est, 1e-3)) + 1))
        for i in range(warmup):
            fn(i)
        ow.check(ow.lib().opw_device_synchronize())
        self._fill(timed)
        self.t0.record(self.stream)
        for i in range(timed):
            fn(i)
        self.t1.record(self.stream)
        self.t1.synchronize()
        ow.check(ow.lib().opw_device_synchronize())
        return self.t0.elapsed_ms(self.t1) / timed


def roofline(achieved: float, peak: float, unit: str, bound: str, traffic=None) -> dict:
    return {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": traffic}


TRAFFIC_FILES = (ROOT / "profiles" / "llama_decode_traffic.md", ROOT / "profiles" / "stream_ops_traffic.md",
                 ROOT / "profiles" / "scan_transpose_gather_traffic.md", ROOT / "profiles" / "gemm_attention_traffic.md",
                 ROOT / "profiles" / "gemm_x6_linear_and_config3.md")


def profiled_traffic(stage: str):
    """HBM bytes per launch of a kernel (a decode stage, or a streaming op's workload name), as measured by
    the committed rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes (scaled by the copy-kernel calibration in
    those files), or None."""
    for path in TRAFFIC_FILES:
        if not path.exists():
            continue
        for line in path.read_text().splitlines():
            if line.startswith(f"traffic_bytes_per_launch {stage}:"):
                return int(line.split(":", 1)[1].strip())
    return None


# ------------------------------------------------------------------ workloads
def wl_map(stream, steps, warmup):
    """Config 2a: ScaleAdd(alpha=2.5) over n = 2^28 fp32; 12 B/element."""
    n = 1 << 28
    a, b, c = (ow.DeviceBuffer.empty(n) for _ in range(3))
    ow.fill_uniform(a, SEED, 0, -1.0, 1.0, stream=stream)
    ow.fill_uniform(b, SEED, 1, -1.0, 1.0, stream=stream)
    ms = Timer(stream).run(lambda i: ow.ops.map_scale_add(a, b, c, n, 2.5, stream=stream), steps, warmup)
    nbytes = 12 * n
    gbs = nbytes / ms / 1e6
    return {"workload": "map_scale_add_n2^28", "unit": "GB/s", "value": gbs, "ms": ms, "bytes": nbytes,
            "kernel": "map_pack_kernel",
            "roofline": roofline(gbs, HBM_PEAK_GBS, "GB/s", "hbm", traffic=profiled_traffic("map"))}


def wl_reduce(stream, steps, warmup):
    """Config 2b: Sum over n = 2^28 fp32 (partial + final launch); 4 B/element."""
    n = 1 << 28
    c = ow.DeviceBuffer.empty(n)
    ow.fill_uniform(c, SEED, 2, -1.0, 1.0, stream=stream)
    out = ow.DeviceBuffer.empty(1)
    ws = ow.DeviceBuffer.empty(ow.ops.reduction_workspace_size(n))
    ms = Timer(stream).run(lambda i: ow.ops.reduce(c, out, n, "sum", ws, stream=stream), steps, warmup)
    nbytes = 4 * n
    gbs = nbytes / ms / 1e6
    return {"workload": "reduce_sum_n2^28", "unit": "GB/s", "value": gbs, "ms": ms, "bytes": nbytes,
            "kernel": "reduce_partial_kernel+reduce_final_kernel",
            "roofline": roofline(gbs, HBM_PEAK_GBS, "GB/s", "hbm", traffic=profiled_traffic("reduce"))}


def _rotating(rows, cols, sets, fill):
    xs, ys = [], []
    for k in range(sets):
        x = ow.DeviceBuffer.empty(rows * cols)
        fill(x, k)
        xs.append(x)
        ys.append(ow.DeviceBuffer.empty(rows * cols))
    return xs, ys


def wl_softmax(stream, steps, warmup):
    """Config 1: softmax rows=4096, cols=1024, x = 4*N(0,1); 8 B/element; 16 rotating buffer pairs (1 GiB)."""
    rows, cols, sets = 4096, 1024, 16
    xs, ys = _rotating(rows, cols, sets, lambda x, k: ow.fill_normal(x, SEED, 100 + k, 0.0, 4.0, stream=stream))
    ms = Timer(stream).run(lambda i: ow.ops.softmax(xs[i % sets], ys[i % sets], rows, cols, stream=stream),
                           steps, warmup)
    nbytes = 8 * rows * cols
    gbs = nbytes / ms / 1e6
    return {"workload": "softmax_4096x1024", "unit": "GB/s", "value": gbs, "ms": ms, "bytes": nbytes,
            "kernel": "softmax_rows_reg_kernel<1,4>",
            "roofline": roofline(gbs, HBM_PEAK_GBS, "GB/s", "hbm", traffic=profiled_traffic("softmax"))}


def wl_rmsnorm(stream, steps, warmup):
    """Config 2c: RMSNorm rows=8192, cols=2048, eps=1e-5, gamma ~ U[0.5,1.5]; 4 rotating pairs (1 GiB)."""
    rows, cols, sets = 8192, 2048, 4
    xs, ys = _rotating(rows, cols, sets, lambda x, k: ow.fill_normal(x, SEED, 200 + k, 0.0, 1.0, stream=stream))
    w = ow.DeviceBuffer.empty(cols)
    ow.fill_uniform(w, SEED, 210, 0.5, 1.5, stream=stream)
    ms = Timer(stream).run(lambda i: ow.ops.rms_norm(xs[i % sets], w, ys[i % sets], rows, cols, 1e-5, stream=stream),
                           steps, warmup)
    nbytes = 8 * rows * cols + 4 * cols
    gbs = nbytes / ms / 1e6
    return {"workload": "rms_norm_8192x2048", "unit": "GB/s", "value": gbs, "ms": ms, "bytes": nbytes,
            "kernel": "rms_norm_reg_kernel<1,8>",
            "roofline": roofline(gbs, HBM_PEAK_GBS, "GB/s", "hbm", traffic=profiled_traffic("rmsnorm"))}


def wl_layernorm(stream, steps, warmup):
    """ops::layer_norm (no configuration names it) at config 2c's shape: rows=8192, cols=2048,
    eps=1e-5, gamma ~ U[0.5,1.5], beta ~ U[-0.1,0.1]; 4 rotating pairs (1 GiB)."""
    rows, cols, sets = 8192, 2048, 4
    xs, ys = _rotating(rows, cols, sets, lambda x, k: ow.fill_normal(x, SEED, 220 + k, 0.0, 1.0, stream=stream))
    g, b = ow.DeviceBuffer.empty(cols), ow.DeviceBuffer.empty(cols)
    ow.fill_uniform(g, SEED, 230, 0.5, 1.5, stream=stream)
    ow.fill_uniform(b, SEED, 231, -0.1, 0.1, stream=stream)
    ms = Timer(stream).run(lambda i: ow.ops.layer_norm(xs[i % sets], ys[i % sets], g, b, rows, cols, 1e-5,
                                                       stream=stream), steps, warmup)
    nbytes = 8 * rows * cols + 8 * cols
    gbs = nbytes / ms / 1e6
    return {"workload": "layer_norm_8192x2048", "unit": "GB/s", "value": gbs, "ms": ms, "bytes": nbytes,
            "kernel": "layer_norm_reg_kernel<1,8>",
            "roofline": roofline(gbs, HBM_PEAK_GBS, "GB/s", "hbm", traffic=profiled_traffic("layernorm"))}


# Timed in a child process that imports only torch: torch's own HIP runtime did not see the GPU
# from a process where this library's runtime already holds it.
LIBRARY_REFERENCE_CHILD = r"""
import json, sys, torch
kind, m, n, k, calls, seed, copies = sys.argv[1], *map(int, sys.argv[2:8])
dev = torch.device("cuda", 0)
g = torch.Generator(device=dev).manual_seed(seed)
# kinds: f32 (A @ B), f32nk (X @ W^T), bf16 (A @ W^T, bf16 result), bf16f32 (A @ W^T, fp32 result);
# A is m x k, the right operand n x k (k x n for f32), rotated over `copies` distinct tensors
dt = torch.bfloat16 if kind.startswith("bf16") else torch.float32
a = (torch.randn(m, k, device=dev, generator=g) / 64).to(dt)
bs = [(torch.randn(k, n, device=dev, generator=g) if kind == "f32" else
       torch.randn(n, k, device=dev, generator=g)).div_(64).to(dt) for _ in range(copies)]
rhs = [b if kind == "f32" else b.t() for b in bs]
out = torch.empty(m, n, device=dev, dtype=torch.float32 if kind == "bf16f32" else dt)
if kind == "bf16f32":
    def call(i):
        torch.mm(a, rhs[i % copies], torch.float32, out=out)
else:
    def call(i):
        torch.matmul(a, rhs[i % copies], out=out)
import time
t_end = time.perf_counter() + 0.3  # back-to-back calls past the clock ramp, as this library's workloads get
while time.perf_counter() < t_end:
    for i in range(10):
        call(i)
    torch.cuda.synchronize()
e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
e0.record()
for i in range(calls):
    call(i)
e1.record()
torch.cuda.synchronize()
print(json.dumps({"ms": e0.elapsed_time(e1) / calls, "torch": torch.__version__}))
"""


def library_reference(kind, n=4096, calls=50, shape=None, copies=1):
    """The vendor library on the same problem, for comparison only (opt-in, --library-reference):
    torch.matmul (hipBLASLt on ROCm) on N(0, 1/64) operands (n^3, or shape = (m, n, k)), `calls`
    back-to-back calls between two events after 0.3 s of untimed ones (the clock ramp), the right
    operand rotated over `copies` tensors. kind "f32": fp32 A @ B; "bf16": bf16 A @ W^T with a bf16
    result (half the output bytes of this library's fp32 result); "bf16f32": bf16 A @ W^T with an fp32
    result (torch.mm's out_dtype, this library's problem); "f32nk": fp32 X @ W^T."""
    import subprocess

    m, nn, k = shape if shape else (n, n, n)
    proc = subprocess.run([sys.executable, "-c", LIBRARY_REFERENCE_CHILD, kind, str(m), str(nn), str(k), str(calls),
                           str(SEED), str(copies)], capture_output=True, text=True, timeout=600)
    if proc.returncode != 0:
        return {"impl": "torch.matmul", "error": proc.stderr.strip().splitlines()[-1:]}
    r = json.loads(proc.stdout.strip().splitlines()[-1])
    ms = r["ms"]
    desc = {"f32": "fp32, A @ B", "f32nk": "fp32, X @ W^T", "bf16": "bf16 in/out, A @ W^T",
            "bf16f32": "bf16 in, fp32 out, A @ W^T"}[kind]
    return {"impl": f"torch {r['torch']} matmul ({desc})",
            "ms": round(ms, 5), "value": round(2.0 * m * nn * k / ms / 1e9, 2), "unit": "TFLOP/s"}


def library_reference_prefill(prompt_len=512):
    """hipBLASLt (torch.mm, bf16 operands, fp32 result) on the bf16 Llama prefill's four projection
    shapes at prompt_len rows, the weights rotated over enough copies (>= 600 MB) that they come
    from HBM as the model's 16 layers' do; microseconds per call."""
    from opworks_amd.llama import LLAMA_3_2_1B as c

    H, I = c["hidden_size"], c["intermediate_size"]
    qkv = (c["num_attention_heads"] + 2 * c["num_key_value_heads"]) * c["head_dim"]
    out = {}
    for name, (n, k) in {"qkv": (qkv, H), "o_proj": (H, c["num_attention_heads"] * c["head_dim"]),
                         "gate_up": (2 * I, H), "down": (H, I)}.items():
        copies = max(2, int(6e8 // (n * k * 2)))
        ref = library_reference("bf16f32", calls=100, shape=(prompt_len, n, k), copies=copies)
        out[name] = round(ref["ms"] * 1e3, 2) if "ms" in ref else ref
    return {"impl": "torch.mm (bf16 in, fp32 out), weights rotated over copies", "rows": prompt_len, "us": out}


def wl_gemm(stream, steps, warmup):
    """Config 3: C = relu(A @ B + bias), M = N = K = 4096 fp32, A, B ~ N(0, 1/64); 2*4096^3 flop."""
    n = 4096
    A, B, C = (ow.DeviceBuffer.empty(n * n) for _ in range(3))
    bias = ow.DeviceBuffer.empty(n)
    ow.fill_normal(A, SEED, 300, 0.0, 1.0 / 64, stream=stream)
    ow.fill_normal(B, SEED, 301, 0.0, 1.0 / 64, stream=stream)
    ow.fill_uniform(bias, SEED, 302, -0.1, 0.1, stream=stream)
    lib = ow.lib()
    ms = Timer(stream).run(lambda i: ow.check(lib.opw_mat_mul_fused_f32(A.ptr, B.ptr, bias.ptr, C.ptr, n, n, n, 0, 1,
                                                                         stream)), steps, warmup)
    flop = 2.0 * n ** 3
    tf = flop / ms / 1e9
    executed = 6.0 * flop / ms / 1e9  # bf16x6 products, as the linear workload's
    return {"workload": "gemm_f32_relu_bias_4096^3", "unit": "TFLOP/s", "value": tf, "ms": ms, "flop": flop,
            "kernel": "gemm_x6_kernel<kn> (bf16x6 products)",
            "roofline": roofline(tf, FP32_PEAK_TFLOPS, "TFLOP/s", "mfma", traffic=profiled_traffic("gemm_x6")),
            "mfma_executed": {"dtype": "bf16", "flop_per_launch": 6.0 * flop, "achieved": round(executed, 2),
                              "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                              "frac": round(executed / BF16_PEAK_TFLOPS, 4)},
            "note": "fp32-accurate products on bf16 MFMAs (three bf16 parts per operand, six MFMAs per product; "
                    "B [K][N] transposed while staged): roofline.frac prices the algorithmic fp32 flops against the "
                    "fp32 MFMA peak and can exceed 1; mfma_executed prices the issued bf16 work against the bf16 "
                    "peak. OPWORKS_GEMM_X6=0 runs the fp32 MFMA kernel instead"}


def wl_gemm_bf16(stream, steps, warmup):
    """Config 3 bf16 variant: relu(A @ W^T + bias), 4096^3, A and W bf16 (RNE-rounded), fp32 accumulate/output."""
    n = 4096
    Af, Wf = ow.DeviceBuffer.empty(n * n), ow.DeviceBuffer.empty(n * n)
    ow.fill_normal(Af, SEED, 300, 0.0, 1.0 / 64, stream=stream)
    ow.fill_normal(Wf, SEED, 301, 0.0, 1.0 / 64, stream=stream)
    A, W = ow.DeviceBuffer.empty(n * n, np.uint16), ow.DeviceBuffer.empty(n * n, np.uint16)
    ow.ops.convert_f32_to_bf16(Af, A, n * n, stream=stream)
    ow.ops.convert_f32_to_bf16(Wf, W, n * n, stream=stream)
    bias, C = ow.DeviceBuffer.empty(n), ow.DeviceBuffer.empty(n * n)
    ow.fill_uniform(bias, SEED, 302, -0.1, 0.1, stream=stream)
    ms = Timer(stream).run(lambda i: ow.ops.linear_bf16(A, W, bias, C, n, n, n, activation="relu", x_bf16=True,
                                                        stream=stream), steps, warmup)
    flop = 2.0 * n ** 3
    tf = flop / ms / 1e9
    return {"workload": "gemm_bf16_relu_bias_4096^3", "unit": "TFLOP/s", "value": tf, "ms": ms, "flop": flop,
            "kernel": "gemm_bf16_mfma_kernel<bf16>",
            "roofline": roofline(tf, BF16_PEAK_TFLOPS, "TFLOP/s", "mfma", traffic=profiled_traffic("gemm_bf16"))}


def wl_linear(stream, steps, warmup):
    """ops::linear at config 3's size: Y = X W^T with X [4096][4096] and W [4096][4096] in the HF
    [out][in] layout (the GEMM's nk form, both operands k-contiguous), fp32, no bias; 2*4096^3 flop."""
    n = 4096
    X, W, Y = (ow.DeviceBuffer.empty(n * n) for _ in range(3))
    ow.fill_normal(X, SEED, 300, 0.0, 1.0 / 64, stream=stream)
    ow.fill_normal(W, SEED, 301, 0.0, 1.0 / 64, stream=stream)
    ms = Timer(stream).run(lambda i: ow.ops.linear(X, W, Y, n, n, n, stream=stream), steps, warmup)
    flop = 2.0 * n ** 3
    tf = flop / ms / 1e9
    # The products run on bf16 MFMAs with both operands in three bf16 parts (six MFMAs per fp32
    # product, fp32 accuracy), as the prefill attention's: `roofline` prices the algorithmic fp32
    # flops against the fp32 MFMA peak, `mfma_executed` the bf16 MFMA work actually issued.
    executed = 6.0 * flop / ms / 1e9
    return {"workload": "linear_f32_4096^3_hf_weights", "unit": "TFLOP/s", "value": tf, "ms": ms, "flop": flop,
            "kernel": "gemm_x6_kernel<nk> (bf16x6 products)",
            "roofline": roofline(tf, FP32_PEAK_TFLOPS, "TFLOP/s", "mfma", traffic=profiled_traffic("linear_x6")),
            "mfma_executed": {"dtype": "bf16", "flop_per_launch": 6.0 * flop, "achieved": round(executed, 2),
                              "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                              "frac": round(executed / BF16_PEAK_TFLOPS, 4)},
            "note": "fp32-accurate products on bf16 MFMAs (three bf16 parts per operand, six MFMAs per product; "
                    "held to the oracle's K-scaled 1e-4 bar, 1.6e-7 of sum |a w| against float64 at this size): "
                    "roofline.frac prices the algorithmic fp32 flops against the fp32 MFMA peak and can exceed 1; "
                    "mfma_executed prices the issued bf16 work against the bf16 peak. OPWORKS_GEMM_X6=0 runs the "
                    "fp32 MFMA kernel instead"}


def wl_attention(stream, steps, warmup):
    """Config 4 prefill: causal GQA 32 q / 8 kv heads, D = 64, T = S = 2048, fp32 N(0,1), scale 1/8.
    Algorithmic flop = 4 * 32 * 64 * (2048 * 2049 / 2) (QK^T and PV over the unmasked triangle)."""
    T, qh, kvh, D = 2048, 32, 8, 64
    q, out = ow.DeviceBuffer.empty(qh * T * D), ow.DeviceBuffer.empty(qh * T * D)
    k, v = ow.DeviceBuffer.empty(kvh * T * D), ow.DeviceBuffer.empty(kvh * T * D)
    ow.fill_normal(q, SEED, 400, 0.0, 1.0, stream=stream)
    ow.fill_normal(k, SEED, 401, 0.0, 1.0, stream=stream)
    ow.fill_normal(v, SEED, 402, 0.0, 1.0, stream=stream)
    ms = Timer(stream).run(lambda i: ow.ops.attention_prefill(q, k, v, out, T, T, 0, qh, 4, D, T, stream=stream),
                           steps, warmup)
    flop = 4.0 * qh * D * (T * (T + 1) / 2)
    tf = flop / ms / 1e9
    # The products run on bf16 MFMAs with every operand in three bf16 parts (six MFMAs per fp32
    # product, fp32 accuracy): `roofline` prices the algorithmic fp32 flops against the fp32 MFMA
    # peak (the work the reference does), `mfma_executed` the bf16 MFMA work actually issued.
    executed = 6.0 * flop / ms / 1e9
    return {"workload": "attention_prefill_causal_gqa_32q8kv_d64_t2048", "unit": "TFLOP/s", "value": tf, "ms": ms,
            "flop": flop, "kernel": "attention_prefill_kernel<4,4,2> (bf16x6 products)",
            "roofline": roofline(tf, FP32_PEAK_TFLOPS, "TFLOP/s", "mfma", traffic=profiled_traffic("attention")),
            "mfma_executed": {"dtype": "bf16", "flop_per_launch": 6.0 * flop, "achieved": round(executed, 2),
                              "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                              "frac": round(executed / BF16_PEAK_TFLOPS, 4)},
            "note": "fp32-accurate products on bf16 MFMAs (three bf16 parts per operand, six MFMAs per product; "
                    "checked against float64 at 2e-6): roofline.frac prices the algorithmic fp32 flops against the "
                    "fp32 MFMA peak and can exceed 1; mfma_executed prices the issued bf16 work against the bf16 peak"}


def wl_attention_decode(stream, steps, warmup):
    """Config 4 decode: one query per head against a 2048-entry cache; 8,404,992 algorithmic bytes.
    The cache is rotated over 32 copies (1 GiB... of K/V) so the Infinity Cache cannot hold it."""
    qh, kvh, D, L, sets = 32, 8, 64, 2048, 32
    q, out = ow.DeviceBuffer.empty(qh * D), ow.DeviceBuffer.empty(qh * D)
    ow.fill_normal(q, SEED, 410, 0.0, 1.0, stream=stream)
    ks, vs = [], []
    for i in range(sets):
        k, v = ow.DeviceBuffer.empty(kvh * L * D), ow.DeviceBuffer.empty(kvh * L * D)
        ow.fill_normal(k, SEED, 411 + 2 * i, 0.0, 1.0, stream=stream)
        ow.fill_normal(v, SEED, 412 + 2 * i, 0.0, 1.0, stream=stream)
        ks.append(k)
        vs.append(v)
    ws_n = ow.ops.attention_decode_workspace_size(qh, L, D)
    ws = ow.DeviceBuffer.empty(ws_n)
    counters = ow.DeviceBuffer.from_host(np.zeros(ow.ops.attention_decode_counters_size(qh, 4), np.int32))
    # the single-launch form (the last chunk workgroup of each kv head merges), as the decode step runs it
    ms = Timer(stream).run(lambda i: ow.ops.attention_decode_fused(q, ks[i % sets], vs[i % sets], out, qh, 4, D, L,
                                                                   L, ws, ws_n, counters, stream=stream),
                           steps, warmup)
    # the two-launch workspace form (partial kernel, then the combine kernel)
    ms_two = Timer(stream).run(lambda i: ow.ops.attention_decode(q, ks[i % sets], vs[i % sets], out, qh, 4, D, L,
                                                                 L, workspace=ws, stream=stream), steps, warmup)
    nbytes = 2 * kvh * L * D * 4 + 2 * qh * D * 4
    gbs = nbytes / ms / 1e6
    return {"workload": "attention_decode_32q8kv_d64_len2048", "unit": "GB/s", "value": gbs, "ms": ms,
            "bytes": nbytes, "kernel": "attention_decode_partial_kernel (fused merge)",
            "two_launch_ms": ms_two, "two_launch_kernels": "attention_decode_partial_kernel+combine",
            "roofline": roofline(gbs, HBM_PEAK_GBS, "GB/s", "hbm", traffic=profiled_traffic("attention_decode"))}


def wl_llama(stream, steps, warmup, bf16=False, prompt_len=512, new_tokens=256, published=None):
    """Config 5: Llama-3.2-1B architecture, fp32 (or bf16) weights N(0, 0.02) (seeded), RMSNorm gamma = 1,
    prompt_len uniform-random prompt ids, greedy new_tokens tokens with the KV cache, no EOS stop. A step
    is one full generation through the C ABI's greedy loop; value = (new_tokens - 1) decode steps / decode
    wall time (median over steps, after warmup). The roofline is the gate/up GEMV (the largest decode
    kernel: 134,266,880 B per launch in fp32) timed with HIP events on the session stream."""
    from opworks_amd.llama import LLAMA_3_2_1B, LlamaModel
    cfg = dict(LLAMA_3_2_1B, torch_dtype="bfloat16") if bf16 else dict(LLAMA_3_2_1B)
    wb = 2 if bf16 else 4  # bytes per weight
    model = LlamaModel.load_random(cfg, SEED, 0.02, "ones")
    sess = model.session(max(1024, prompt_len + new_tokens))
    rng = np.random.default_rng(SEED)
    prompt = [int(v) for v in rng.integers(0, cfg["vocab_size"], prompt_len)]
    runs = []
    for i in range(warmup + steps):
        sess.reset()
        toks, pre_ms, dec_ms = sess.generate_greedy(prompt, new_tokens)
        if i >= warmup:
            runs.append((pre_ms, dec_ms, toks))
    dec = sorted(r[1] for r in runs)[len(runs) // 2]
    pre = sorted(r[0] for r in runs)[len(runs) // 2]
    tok_s = (new_tokens - 1) / (dec / 1e3)
    # The reference's own method (scripts/llama/benchmark.py:53-68): reset, prefill, then one
    # opw_llama_decode_step call per token from the host (a round trip and a synchronize each);
    # median of the per-run decode rates. The ids must equal the chained generation's.
    loop_rates = []
    for i in range(2 + min(steps, 5)):
        sess.reset()
        tok = sess.prefill(prompt)
        ids = [tok]
        t0 = time.perf_counter()
        for _ in range(new_tokens - 1):
            tok = sess.decode_step(tok)
            ids.append(tok)
        t1 = time.perf_counter()
        if ids != [int(t) for t in runs[-1][2]]:
            raise RuntimeError("per-token decode_step loop and chained generation produced different ids")
        if i >= 2:
            loop_rates.append((new_tokens - 1) / (t1 - t0))
    loop_tok_s = sorted(loop_rates)[len(loop_rates) // 2]
    # Each decode stage launched back to back over the 16 layers (HIP events on the session stream):
    # kernel time without launch gaps, comparable with rocprofv3's per-kernel average.
    H, I, V, L = cfg["hidden_size"], cfg["intermediate_size"], cfg["vocab_size"], cfg["num_hidden_layers"]
    qkv_w = (cfg["num_attention_heads"] + 2 * cfg["num_key_value_heads"]) * cfg["head_dim"]
    kernel_bytes = {"qkv_rope": wb * qkv_w * H + 4 * 2 * H, "o_proj": wb * H * H + 4 * 3 * H,
                    "gate_up": wb * 2 * I * H + 4 * (2 * H + I), "down": wb * H * I + 4 * (I + 2 * H),
                    "lm_head": wb * V * H + 4 * (2 * H + V)}
    breakdown = {}
    for k in sess.STAGES:
        us = sess.time_decode_stage(k, reps=10)
        entry = {"avg_us": round(us, 2)}
        if k in kernel_bytes:
            entry["gbs"] = round(kernel_bytes[k] / (us * 1e-6) / 1e9, 1)
        breakdown[k] = entry
    gu_gbs = kernel_bytes["gate_up"] / (breakdown["gate_up"]["avg_us"] * 1e-6) / 1e9
    weight_bytes = wb * (V * H + L * (qkv_w * H + H * H + 2 * I * H + H * I)) + 4 * (2 * L + 1) * H
    kv_bytes_avg = 2 * L * cfg["num_key_value_heads"] * cfg["head_dim"] * 4 * (prompt_len + new_tokens / 2)
    step_gbs = (weight_bytes + kv_bytes_avg) / (dec / (new_tokens - 1) * 1e-3) / 1e9
    out = {"workload": f"llama3.2-1b_{'bf16' if bf16 else 'fp32'}_greedy_prompt{prompt_len}_gen{new_tokens}",
           "unit": "tok/s", "value": tok_s,
           "ms": pre + dec, "ttft_ms": round(pre, 3), "decode_ms_per_token": round(dec / (new_tokens - 1), 4),
           "kernel": f"swiglu_gemv_kernel<8{', bf16' if bf16 else ''}> (gate/up)",
           "roofline": roofline(gu_gbs, HBM_PEAK_GBS, "GB/s", "hbm",
                                traffic=profiled_traffic("bf16_gate_up" if bf16 else "gate_up")),
           # the whole step's counted bytes exist for the configuration they were measured on
           "decode_step_roofline": roofline(step_gbs, HBM_PEAK_GBS, "GB/s", "hbm",
                                            traffic=profiled_traffic("bf16_decode_step")
                                            if bf16 and (prompt_len, new_tokens) == (512, 128) else None),
           "decode_step_loop_tok_s": round(loop_tok_s, 2),
           "decode_step_loop_method": "reference scripts/llama/benchmark.py:53-68: one opw_llama_decode_step "
                                      "call per token from the host, median of the runs",
           "weight_bytes_per_token": weight_bytes, "kernels": breakdown,
           "first_tokens": [int(t) for t in runs[-1][2][:8]]}
    if published:  # the reference's own figure for this exact configuration (other hardware)
        out["published"] = published
        out["vs_published"] = round(tok_s / published["decode_tok_s"], 2)
        if "ttft_ms" in published:
            out["ttft_vs_published"] = round(published["ttft_ms"] / pre, 2)
    return out


def wl_scan(stream, steps, warmup):
    """ScanBuilder's kernel: inclusive prefix sum over n = 2^28 fp32. Algorithmic bytes 8 B/element (read x,
    write out); the one-pass design moves the same 8, plus the published totals (8 B per
    16384-element unit) and a small workspace clear."""
    n = 1 << 28
    x = ow.DeviceBuffer.empty(n)
    ow.fill_uniform(x, SEED, 3, -1.0, 1.0, stream=stream)
    out = ow.DeviceBuffer.empty(n)
    ws_n = ow.ops.scan_workspace_size(n)
    ws = ow.DeviceBuffer.empty(ws_n)
    ms = Timer(stream).run(lambda i: ow.ops.scan(x, out, n, "sum", True, ws, ws_n, stream=stream), steps, warmup)
    nbytes = 8 * n
    gbs = nbytes / ms / 1e6
    return {"workload": "scan_sum_inclusive_n2^28", "unit": "GB/s", "value": gbs, "ms": ms, "bytes": nbytes,
            "moved_bytes": 8 * n, "kernel": "scan_clear_kernel+scan_pair_kernel",
            "roofline": roofline(gbs, HBM_PEAK_GBS, "GB/s", "hbm", traffic=profiled_traffic("scan"))}


def wl_transpose(stream, steps, warmup):
    """TransformBuilder's transpose: 8192 x 8192 fp32 (256 MiB each way), two buffer pairs rotated;
    8 B/element."""
    rows = cols = 8192
    xs, ys = _rotating(rows, cols, 2, lambda b, k: ow.fill_uniform(b, SEED, 30 + k, -1.0, 1.0, stream=stream))
    ms = Timer(stream).run(lambda i: ow.ops.transpose(xs[i % 2], ys[i % 2], rows, cols, stream=stream), steps,
                           warmup)
    nbytes = 8 * rows * cols
    gbs = nbytes / ms / 1e6
    return {"workload": "transpose_8192x8192", "unit": "GB/s", "value": gbs, "ms": ms, "bytes": nbytes,
            "kernel": "transpose_kernel<true>",
            "roofline": roofline(gbs, HBM_PEAK_GBS, "GB/s", "hbm", traffic=profiled_traffic("transpose"))}


def wl_gather(stream, steps, warmup):
    """GatherScatterBuilder's gather: out[i] = in[idx[i]] over n = 2^26 with a random permutation;
    12 B/element algorithmic (index, source element, output). The source side is random, so each
    element costs a whole memory sector there."""
    n = 1 << 26
    x = ow.DeviceBuffer.empty(n)
    ow.fill_uniform(x, SEED, 40, -1.0, 1.0, stream=stream)
    idx = ow.DeviceBuffer.from_host(np.random.default_rng(SEED).permutation(n).astype(np.int32), dtype=np.int32)
    out = ow.DeviceBuffer.empty(n)
    ms = Timer(stream).run(lambda i: ow.ops.gather(x, n, idx, out, n, stream=stream), steps, warmup)
    nbytes = 12 * n
    gbs = nbytes / ms / 1e6
    return {"workload": "gather_random_permutation_n2^26", "unit": "GB/s", "value": gbs, "ms": ms,
            "bytes": nbytes, "kernel": "gather_kernel<true>",
            "roofline": roofline(gbs, HBM_PEAK_GBS, "GB/s", "hbm", traffic=profiled_traffic("gather"))}


WORKLOADS = {"map": wl_map, "reduce": wl_reduce, "softmax": wl_softmax, "rmsnorm": wl_rmsnorm, "layernorm": wl_layernorm, "gemm": wl_gemm, "gemm_bf16": wl_gemm_bf16, "linear": wl_linear, "attention": wl_attention,
             "attention_decode": wl_attention_decode, "scan": wl_scan, "transpose": wl_transpose,
             "gather": wl_gather, "llama": wl_llama,
             # the reference's published configurations (README.md:320-339, RTX 4080 SUPER, 128 new tokens)
             "llama_fp32_p128": lambda st, k, w: wl_llama(
                 st, k, w, prompt_len=128, new_tokens=128,
                 published={"decode_tok_s": 127, "hardware": "RTX 4080 SUPER", "source": "README.md:338-339"}),
             "llama_bf16": lambda st, k, w: wl_llama(
                 st, k, w, bf16=True, prompt_len=512, new_tokens=128,
                 published={"decode_tok_s": 215, "ttft_ms": 103.5, "hardware": "RTX 4080 SUPER",
                            "source": "README.md:320-326"}),
             # the reference's long-prompt rows of the same table (bf16, 128 new tokens)
             "llama_bf16_p1024": lambda st, k, w: wl_llama(
                 st, min(k, 10), min(w, 2), bf16=True, prompt_len=1024, new_tokens=128,
                 published={"decode_tok_s": 198, "ttft_ms": 183.9, "hardware": "RTX 4080 SUPER",
                            "source": "README.md:324"}),
             "llama_bf16_p4096": lambda st, k, w: wl_llama(
                 st, min(k, 6), min(w, 2), bf16=True, prompt_len=4096, new_tokens=128,
                 published={"decode_tok_s": 134, "ttft_ms": 711.3, "hardware": "RTX 4080 SUPER",
                            "source": "README.md:325"}),
             "llama_bf16_p8000": lambda st, k, w: wl_llama(
                 st, min(k, 4), min(w, 1), bf16=True, prompt_len=8000, new_tokens=128,
                 published={"decode_tok_s": 95, "ttft_ms": 1874.3, "hardware": "RTX 4080 SUPER",
                            "source": "README.md:326"})}
HEADLINE = "llama"


# --------------------------------------------------------------- CPU baseline
CPU_SAMPLES = ("map", "reduce", "softmax", "rmsnorm", "layernorm", "gemm", "gemm_bf16", "linear", "attention", "attention_decode", "scan",
               "transpose", "gather", "llama", "llama_bf16")


def host_cpu() -> dict:
    """The host the CPU baseline runs on: model name, what the OS reports, what this run may use."""
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count() or 1
    return {"model": model, "nproc": os.cpu_count(), "affinity": affinity, "threads_used": cpu_threads(),
            "thread_cap": "16 threads: the GPU pool's CPU share per GPU, whatever nproc reports"}


def _rate(fn, budget_s: float, max_reps: int = 1 << 30):
    """Repeats fn for about budget_s of wall time; returns (reps, seconds per call)."""
    reps, t0 = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        if time.perf_counter() - t0 > budget_s or reps >= max_reps:
            return reps, (time.perf_counter() - t0) / reps


def _cpu_work(name: str):
    """(fn, units per call, unit, sample description, budget s) for the oracle on a bounded sample of a workload."""
    from tests import oracle as orc

    if name == "map":
        n = 1 << 26
        a = orc.fill_uniform(n, SEED, 0, -1, 1, mt=True)
        b = orc.fill_uniform(n, SEED, 1, -1, 1, mt=True)
        return (lambda: orc.map_scale_add(a, b, 2.5, mt=True), 12 * n / 1e9, "GB/s",
                "oracle orc_map_scale_add over n=2^26 (768 MiB)", 5.0)
    if name == "reduce":
        n = 1 << 24
        x = orc.fill_uniform(n, SEED, 2, -1, 1, mt=True)
        return (lambda: orc.reduce(x, "sum"), 4 * n / 1e9, "GB/s",
                "oracle orc_reduce (the reference's block order; blocks split across threads) over n=2^24", 3.0)
    if name == "softmax":
        rows, cols = 1024, 1024
        x = orc.fill_normal(rows * cols, SEED, 100, 0, 4, mt=True)
        return (lambda: orc.softmax_rows(x, rows, cols), 8 * rows * cols / 1e9, "GB/s",
                "oracle orc_softmax_rows, 1024 of the 4096 rows", 3.0)
    if name in ("rmsnorm", "layernorm"):
        rows, cols = 2048, 2048
        x = orc.fill_normal(rows * cols, SEED, 200, 0, 1, mt=True)
        g = orc.fill_uniform(cols, SEED, 210, 0.5, 1.5)
        bt = orc.fill_uniform(cols, SEED, 231, -0.1, 0.1)
        fn = ((lambda: orc.rms_norm_rows(x, g, rows, cols, 1e-5)) if name == "rmsnorm"
              else (lambda: orc.layer_norm_rows(x, g, bt, rows, cols, 1e-5)))
        return (fn, 8 * rows * cols / 1e9, "GB/s", f"oracle orc_{'rms' if name == 'rmsnorm' else 'layer'}_norm_rows, "
                "2048 of the 8192 rows", 3.0)
    if name in ("gemm", "gemm_bf16"):
        n, sample = 4096, np.arange(0, 4096, 64)
        A = orc.fill_normal(n * n, SEED, 300, 0.0, 1.0 / 64, mt=True)
        B = orc.fill_normal(n * n, SEED, 301, 0.0, 1.0 / 64, mt=True)
        bias = orc.fill_uniform(n, SEED, 302, -0.1, 0.1)
        if name == "gemm_bf16":  # the reference's CPU check of the bf16 path: fp32 math on rounded inputs
            A, B = orc.round_bf16(A)[0], orc.round_bf16(B)[0]
        return (lambda: orc.mat_mul_rows(A, B, n, n, n, rows=sample, bias=bias, act="relu"),
                2.0 * len(sample) * n * n / 1e12, "TFLOP/s",
                f"oracle orc_mat_mul_rows (fp32, plus its float64 |a·b| bound), {len(sample)} of the 4096 rows of "
                "relu(A·B+bias)", 3.0)
    if name == "linear":
        n, sample = 4096, np.arange(0, 4096, 64)
        X = orc.fill_normal(n * n, SEED, 300, 0.0, 1.0 / 64, mt=True)
        W = orc.fill_normal(n * n, SEED, 301, 0.0, 1.0 / 64, mt=True)
        return (lambda: orc.mat_mul_rows(X, W, n, n, n, rows=sample, b_transposed=True),
                2.0 * len(sample) * n * n / 1e12, "TFLOP/s",
                f"oracle orc_mat_mul_rows (fp32, W in [out][in]), {len(sample)} of the 4096 rows of X W^T", 3.0)
    if name == "attention":
        T, qh, kvh, D = 2048, 32, 8, 64
        q = orc.fill_normal(qh * T * D, SEED, 400, 0.0, 1.0, mt=True)
        k = orc.fill_normal(kvh * T * D, SEED, 401, 0.0, 1.0, mt=True)
        v = orc.fill_normal(kvh * T * D, SEED, 402, 0.0, 1.0, mt=True)
        rows = np.arange(0, T, 128)
        flop = 4.0 * qh * D * float(np.sum(rows + 1))  # unmasked QK^T + PV of the sampled causal rows
        return (lambda: orc.attention_explicit(q, k, v, T, T, qh, 4, D, T, rows=rows), flop / 1e12, "TFLOP/s",
                f"oracle orc_attention_explicit, {len(rows)} of the 2048 causal query rows of every head "
                "(unmasked flops)", 3.0)
    if name == "attention_decode":
        qh, kvh, D, L = 32, 8, 64, 2048
        q = orc.fill_normal(qh * D, SEED, 410, 0.0, 1.0)
        k = orc.fill_normal(kvh * L * D, SEED, 411, 0.0, 1.0, mt=True)
        v = orc.fill_normal(kvh * L * D, SEED, 412, 0.0, 1.0, mt=True)
        return (lambda: orc.attention_decode(q, k, v, qh, 4, D, L, L), (2 * kvh * L * D * 4 + 2 * qh * D * 4) / 1e9,
                "GB/s", "oracle orc_attention_decode (q heads split across threads), the full config (len 2048)", 3.0)
    if name == "scan":
        n = 1 << 24
        x = orc.fill_uniform(n, SEED, 500, -1.0, 1.0, mt=True)
        return (lambda: orc.scan(x), 8 * n / 1e9, "GB/s",
                "oracle orc_scan (inclusive sum in index order, with its float64 |x| prefix: sequential by "
                "definition, so one thread at any count) over n=2^24", 3.0)
    if name == "transpose":
        r = c = 4096
        x = orc.fill_uniform(r * c, SEED, 510, -1.0, 1.0, mt=True)
        return (lambda: orc.transpose(x, r, c), 8 * r * c / 1e9, "GB/s",
                "oracle orc_transpose of 4096x4096 (a quarter of the 8192x8192 config)", 3.0)
    if name == "gather":
        n = 1 << 24
        x = orc.fill_uniform(n, SEED, 520, -1.0, 1.0, mt=True)
        idx = np.random.default_rng(SEED).permutation(n).astype(np.int32)
        return (lambda: orc.gather(x, idx), 12 * n / 1e9, "GB/s",
                "oracle orc_gather through a random permutation of 2^24", 3.0)
    return None


def _cpu_llama(name: str, threads: int) -> dict:
    """The oracle's Llama forward on the same seeded weights: all-threads and single-thread greedy decode."""
    from tests import oracle as orc
    from opworks_amd.llama import LLAMA_3_2_1B
    cfg = dict(LLAMA_3_2_1B, torch_dtype="bfloat16") if name == "llama_bf16" else dict(LLAMA_3_2_1B)
    orc.set_threads(threads)
    t_build = time.perf_counter()
    model = orc.Llama(cfg, SEED, 0.02, "ones")
    build_s = time.perf_counter() - t_build
    prompt = [int(v) for v in np.random.default_rng(SEED).integers(0, cfg["vocab_size"], 512)]
    out = {}
    for label, nthreads, plen, budget, cap in (("all", threads, 16, 15.0, 64), ("one", 1, 2, 8.0, 16)):
        orc.set_threads(nthreads)
        model.reset(1024)
        tok, _ = model.prefill(prompt[:plen])
        steps, t0 = 0, time.perf_counter()
        while True:
            tok, _ = model.decode(tok)
            steps += 1
            if time.perf_counter() - t0 > budget or steps >= cap:
                break
        out[label] = (round(steps / (time.perf_counter() - t0), 3), steps, plen)
    del model
    orc.set_threads(threads)
    kind = "bf16-weight" if name == "llama_bf16" else "fp32"
    return {"value": out["all"][0], "unit": "tok/s", "cores": threads, "kind": "port",
            "single_thread": {"value": out["one"][0], "cores": 1},
            "sample": f"oracle {kind} Llama forward (orc_llama_*), same seeded weights; all threads: "
                      f"{out['all'][2]}-token prompt then {out['all'][1]} greedy decode steps timed (~15 s); one "
                      f"thread: {out['one'][2]}-token prompt then {out['one'][1]} steps (~8 s); weight generation "
                      f"{build_s:.1f} s untimed",
            "host": host_cpu()}


SERIAL_ORACLE = ("scan",)  # oracle functions that do not split over threads


def cpu_baseline(name: str) -> dict:
    """Times the oracle on a bounded sample of the same workload on this host, with every thread this
    run may use and with one thread."""
    from tests import oracle as orc

    threads = cpu_threads()
    if name in ("llama", "llama_bf16"):
        return _cpu_llama(name, threads)
    orc.set_threads(threads)
    work = _cpu_work(name)
    if work is None:
        return {}
    fn, units, unit, sample, budget = work
    digits = 6 if unit == "TFLOP/s" else 3
    if name in SERIAL_ORACLE:  # one thread whatever set_threads says: report it as such
        reps, dt = _rate(fn, budget)
        return {"value": round(units / dt, digits), "unit": unit, "cores": 1, "kind": "port",
                "sample": f"{sample}; {reps} reps, single-threaded oracle function", "host": host_cpu()}
    reps, dt = _rate(fn, budget)
    orc.set_threads(1)
    reps1, dt1 = _rate(fn, budget / 2)
    orc.set_threads(threads)
    return {"value": round(units / dt, digits), "unit": unit, "cores": threads, "kind": "port",
            "single_thread": {"value": round(units / dt1, digits), "cores": 1},
            "sample": f"{sample}; {reps} reps on {threads} threads, {reps1} on one", "host": host_cpu()}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="all", help="all | " + " | ".join(WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--library-reference", action="store_true",
                    help="also time torch.matmul (hipBLASLt) beside the gemm, gemm_bf16 and linear workloads, "
                         "and on the bf16 prefill's projection shapes beside llama_bf16")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only; --gpus {args.gpus} is not supported "
              "(the path has no multi-GPU component; see DESIGN.md for how it would shard)", file=sys.stderr)
        return 2
    names = list(WORKLOADS) if args.workload == "all" else args.workload.split(",")
    headline = HEADLINE if HEADLINE in names else names[0]
    stream = ow.Stream()
    results = {}
    for name in names:
        results[name] = WORKLOADS[name](stream.handle, args.steps, args.warmup)
        print(f"[bench] {name}: {results[name]['value']:.1f} {results[name]['unit']} "
              f"({results[name]['ms']:.4f} ms/step)", file=sys.stderr, flush=True)
    if args.library_reference:  # after every workload of this library, so it cannot disturb them
        for name, kind, key in (("gemm", "f32", "library_reference"), ("gemm_bf16", "bf16f32", "library_reference"),
                                ("gemm_bf16", "bf16", "library_reference_bf16_out"),
                                ("linear", "f32nk", "library_reference")):
            if name in results:
                ref = library_reference(kind)
                if "value" in ref:
                    ref["ratio"] = round(results[name]["value"] / ref["value"], 4)  # this library / the vendor's
                results[name][key] = ref
                print(f"[bench] {name} {key}: {ref.get('value', ref.get('error'))}", file=sys.stderr, flush=True)
        if "llama_bf16" in results:  # the prefill's projection GEMMs against the library's
            results["llama_bf16"]["library_reference_prefill"] = library_reference_prefill()
            print(f"[bench] llama_bf16 library_reference_prefill: "
                  f"{results['llama_bf16']['library_reference_prefill']['us']}", file=sys.stderr, flush=True)
    if not args.no_cpu:  # the oracle on this host beside every GPU figure (bounded samples)
        for name in names:
            if name != headline and name in CPU_SAMPLES:
                results[name]["cpu_baseline"] = cpu_baseline(name)
                print(f"[bench] {name} cpu: {results[name]['cpu_baseline']['value']} "
                      f"{results[name]['cpu_baseline']['unit']}", file=sys.stderr, flush=True)
    head = results[headline]
    line = {
        "metric": METRIC,
        "value": round(head["value"], 2),
        "unit": head["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (counter-based seeded generator, seed 1234, resident in HBM)",
        "config": {"workload": head["workload"], "device": ow.device_name()},
        "roofline": head["roofline"],
        # the whole decode step against the weight-streaming bound (weights + KV cache bytes per token)
        "decode_step_roofline": head.get("decode_step_roofline"),
        "cpu_baseline": None if args.no_cpu else cpu_baseline(headline),
        "components": {k: {kk: (round(vv, 5) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                       for k, v in results.items()},
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
