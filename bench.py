"""Benchmark of the quantized DiT hot path on one MI355X (gfx950).

Metric: INT8 TOPS + % MFMA peak, W8A8 GEMM & Sage attention at
Wan-14B shapes, 1 GPU.

One step = the Wan-14B block's hot path on synthetic inputs already resident
in HBM:
  * the four ConvRot W8A8 linears of config 4 (M=32760 tokens; qkv K5120 N15360,
    out K5120 N5120, ffn-up K5120 N13824, ffn-down K13824 N5120), each = ConvRot
    quantize (G=128) + INT8 GEMM with the per-token x per-channel epilogue;
  * Sage attention of config 3 (B1 H40 L32760 D128): K mean, Q/K per-128-token
    INT8 quantization, INT8 QK^T + online softmax + bf16 PV.
value = (sum of 2MNK over the linears + 4 B H L^2 D) / step time, in TOPS.

Per-kernel average durations come from HIP events recorded on torch's current
stream, which is the stream every op of this package launches on, inside the
timed region.  The roofline entry is for the kernel with the largest total
time; its ``mfma_busy`` and ``clock_ghz`` come from profiles/mfma_counters.json
(rocprofv3 --pmc passes of this script) and its ``traffic`` from
profiles/traffic.json: the bytes per launch
the L2 requested from the fabric (rocprofv3 --pmc passes of this script over
TCC_EA0_RDREQ_{32B,64B,128B} / TCC_EA0_WRREQ{,_64B}, request counts times their
sizes; FETCH_SIZE / WRITE_SIZE scaled by ``--copy-calibration``'s 1 GiB copy
agree within 1.3 %), an upper bound on HBM bytes since the Infinity Cache may
serve part of them.
cpu_baseline times the reference's CPU path -- its PyTorch fallback: bf16
linear on the dequantized weight and bf16 scaled_dot_product_attention -- on a
bounded sample of the same workload on this host's cores; the CPU oracle
(oracle/, a plain-C restatement of the reference arithmetic) is reported
beside it on the same sample.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
                       [--cpu-seconds S] [--copy-calibration] [--no-extras] [--power-probe]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "comfyui-turing-utils_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_INT8_TOPS = 5000.0     # MI355X published dense INT8 MFMA, 5.0 POP/s
PEAK_BF16_TFLOPS = 2500.0   # MI355X published dense BF16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E, 8 TB/s
M_TOKENS = 32760
LINEARS = (("qkv", 5120, 15360), ("out", 5120, 5120), ("ffn_up", 5120, 13824), ("ffn_down", 13824, 5120))
ATTN = dict(b=1, h=40, l=32760, d=128)
GROUP = 128
BLK = 128


def parse_args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=30.0, help="approximate CPU baseline budget (s)")
    p.add_argument("--copy-calibration", action="store_true",
                   help="after the timed steps, copy 1 GiB once (HBM-counter calibration for rocprofv3 --pmc)")
    p.add_argument("--no-extras", action="store_true",
                   help="skip the next-row kernels timed outside the step (short runs under rocprofv3 --pmc)")
    p.add_argument("--power-probe", action="store_true",
                   help="only time the qkv GEMM and the attention kernel on the bench inputs and on all-zero "
                        "operands of the same shapes (three launches each), print one JSON line and exit")
    return p.parse_args()


class KernelTimer:
    """Pairs of HIP events around launches on the current stream, per kernel name."""

    def __init__(self, torch):
        self.torch = torch
        self.pending = []
        self.enabled = False

    def __call__(self, name, fn, *args, **kwargs):
        if not self.enabled:
            return fn(*args, **kwargs)
        start = self.torch.cuda.Event(enable_timing=True)
        end = self.torch.cuda.Event(enable_timing=True)
        start.record()
        out = fn(*args, **kwargs)
        end.record()
        self.pending.append((name, start, end))
        return out

    def summary(self, steps):
        totals = {}
        counts = {}
        for name, s, e in self.pending:
            totals[name] = totals.get(name, 0.0) + s.elapsed_time(e)
            counts[name] = counts.get(name, 0) + 1
        return {n: {"ms_avg": totals[n] / counts[n], "ms_per_step": totals[n] / steps, "launches": counts[n]}
                for n in totals}


def main():
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the hot path shards by tokens for the linears and by heads for the attention, "
              "with no exchange between GPUs). "
              "Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    import comfyui_turing_utils_kernel  # noqa: F401  (registers torch.ops.turing_utils.*)
    from comfyui_turing_utils_kernel import _lib
    from comfyui_turing_utils_kernel.turing_sage import quant as sage_quant
    from comfyui_turing_utils_kernel.turing_sage.core import attention_from_vt
    from tests import inputs

    dev = torch.device("cuda", 0)
    if not _lib.device_supported(dev):
        raise SystemExit(f"bench.py needs a gfx950 GPU, got {torch.cuda.get_device_name(0)}")
    torch.cuda.set_device(dev)

    # ---- synthetic inputs, generated on the CPU with fixed seeds, then moved to HBM
    lin = []
    for idx, (name, k, n) in enumerate(LINEARS):
        x = inputs.activation(M_TOKENS, k, 3 + idx).to(dev)
        w, ws, _ = inputs.weights(n, k, 3 + idx, with_bias=False)
        lin.append((name, k, n, x, w.to(dev), ws.to(dev)))
    q, k_, v = (t.to(dev) for t in inputs.attention(ATTN["b"], ATTN["h"], ATTN["l"], ATTN["d"], 2))
    torch.cuda.synchronize()

    timer = KernelTimer(torch)
    ops = torch.ops.turing_utils
    sm_scale = ATTN["d"] ** -0.5
    if args.power_probe:
        print(json.dumps(power_probe(torch, ops, lin[0], q, k_, v)))
        return 0

    def step():
        for name, _, _, x, w, ws in lin:
            qa, sa = timer(f"convrot_quant_k{x.shape[1]}", ops.bf16_int8_convrot_quantize, x, GROUP)
            timer(f"int8_gemm_{name}", ops.int8_linear, qa, w, sa, ws, None)
        mean = timer("sage_kmean", sage_quant.key_channel_mean, k_, "HND")
        q8, qs = timer("sage_quant_q", sage_quant.quantize_per_block, q, BLK, "HND")
        k8, ks = timer("sage_quant_k", sage_quant.quantize_per_block, k_, BLK, "HND", mean)
        vt, _ = timer("sage_v_prep", sage_quant.value_transpose, v, "HND")
        return timer("sage_attn", attention_from_vt, q8, qs, k8, ks, vt, tensor_layout="HND",
                     sm_scale=sm_scale, blkq=BLK, blkk=BLK)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    timer.enabled = True
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_per_step = (t1 - t0) * 1e3 / args.steps
    kernels = timer.summary(args.steps)
    copy_gbs = copy_bandwidth(torch, dev)
    if args.copy_calibration:
        # one elementwise kernel that reads and writes exactly 1 GiB: the
        # reference point for the byte counters
        src = torch.ones(1 << 28, dtype=torch.int32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst

    lin_ops = sum(2.0 * M_TOKENS * n * k for _, k, n, *_ in lin)
    attn_ops = 4.0 * ATTN["b"] * ATTN["h"] * ATTN["l"] ** 2 * ATTN["d"]
    total_ops = lin_ops + attn_ops
    value = total_ops / (ms_per_step * 1e-3) / 1e12

    # Per-kernel algorithmic work: GEMM 2MNK ops; attention 4BHL^2D ops;
    # ConvRot quantize 2 B/elem read + 1 B/elem write + 4 B/row; Sage quantize
    # 2 B read + 1 B write per element (K also reads its mean: negligible);
    # K mean 2 B/elem read; V transpose 2 B read + 2 B write per element.
    work = {}
    for name, k, n, *_ in lin:
        work[f"int8_gemm_{name}"] = ("mfma", 2.0 * M_TOKENS * n * k)
        work[f"convrot_quant_k{k}"] = ("hbm", 3.0 * M_TOKENS * k + 4.0 * M_TOKENS)
    elems = ATTN["b"] * ATTN["h"] * ATTN["l"] * ATTN["d"]
    work["sage_attn"] = ("mfma", attn_ops)
    work["sage_quant_q"] = ("hbm", 3.0 * elems)
    work["sage_quant_k"] = ("hbm", 3.0 * elems)
    work["sage_kmean"] = ("hbm", 2.0 * elems)
    work["sage_v_prep"] = ("hbm", 4.0 * elems)
    for name, rec in kernels.items():
        bound, amount = work[name]
        sec = rec["ms_avg"] * 1e-3
        if bound == "mfma":
            rec["tops"] = amount / sec / 1e12
            rec["frac_int8_peak"] = rec["tops"] / PEAK_INT8_TOPS
        else:
            rec["gbs"] = amount / sec / 1e9
            rec["frac_hbm_peak"] = rec["gbs"] / PEAK_HBM_GBS
            rec["frac_copy"] = rec["gbs"] / copy_gbs
    # attention: half its ops are INT8 (QK^T), half BF16 (PV); time at the
    # mixed peak relative to the measured time
    rec = kernels["sage_attn"]
    rec["frac_mixed_peak"] = (attn_ops / 2 / (PEAK_INT8_TOPS * 1e12) + attn_ops / 2 / (PEAK_BF16_TFLOPS * 1e12)) / (
        rec["ms_avg"] * 1e-3)
    dominant = max(kernels, key=lambda n: kernels[n]["ms_per_step"])
    bound, amount = work[dominant]
    achieved = kernels[dominant]["tops"] if bound == "mfma" else kernels[dominant]["gbs"]
    peak = PEAK_INT8_TOPS if bound == "mfma" else PEAK_HBM_GBS
    roofline = {
        "kernel": dominant,
        "bound": bound,
        "achieved": achieved,
        "peak": peak,
        "unit": "TFLOP/s" if bound == "mfma" else "GB/s",
        "frac": achieved / peak,
        "traffic": None,
    }
    # committed rocprofv3 figures of the same kernel and workload, used only
    # when they were captured from that kernel's sources in this tree
    traffic_src, mfma_src = counters_source(TRAFFIC_FILE, dominant), counters_source(MFMA_FILE, dominant)
    if traffic_src["current"]:
        roofline["traffic"] = measured_traffic(dominant)
    counters = measured_mfma(dominant) if mfma_src["current"] else None
    if bound == "mfma" and counters is not None:
        roofline["mfma_busy"] = counters["mfma_busy"]
        roofline["clock_ghz"] = counters["clock_ghz"]
    roofline["counters_source"] = {"traffic": traffic_src, "mfma": mfma_src}

    extras = None if args.no_extras else extra_kernels(torch, dev, ops, lin, q, k_, v, copy_gbs)
    if extras is not None:
        extras["power_probe"] = power_probe(torch, ops, lin[0], q, k_, v)
    cpu = None if args.no_cpu_baseline else cpu_baseline(args.cpu_seconds)

    record = {
        "metric": "INT8 TOPS + % MFMA peak: W8A8 GEMM & Sage attn at Wan-14B shapes, 1 GPU",
        "value": value,
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded Wan-14B shapes: 0.1% x20 outlier channels; int8 weights; "
                "K per-head channel bias), inputs resident in HBM",
        "config": {
            "workload": "wan14b_block_hot_path: 4x ConvRot W8A8 linear (config 4, M=32760, G=128) "
                        "+ Sage INT8 attention (config 3, B1 H40 L32760 D128, BLKQ=BLKK=128, K-smoothing)",
            "linears": [{"name": n, "M": M_TOKENS, "K": k, "N": nn} for n, k, nn, *_ in lin],
            "attention": ATTN,
            "ops_per_step": total_ops,
        },
        "kernels": kernels,
        "extra_kernels": extras,
        "roofline": roofline,
        "hbm_copy_gbs": copy_gbs,
        "cpu_baseline": cpu,
    }
    print(json.dumps(record))
    return 0


def power_probe(torch, ops, qkv, q, k, v) -> dict:
    """The qkv GEMM and the attention kernel, each launched three times on the
    bench inputs and three times on all-zero operands of the same shapes (the
    scales and the launch are unchanged).  The GEMM runs the same instruction
    stream either way (its only data-dependent branch, the epilogue's
    finiteness test, takes the same side); the attention's rescale test is
    rarely taken on either.  So a shorter time on zeros is a higher clock:
    multipliers and buses that do not toggle draw less power, and MI355X
    holds these loops at its board power limit on the bench data."""
    from comfyui_turing_utils_kernel.turing_sage import quant as sage_quant
    from comfyui_turing_utils_kernel.turing_sage.core import attention_from_vt

    def timed(fn, reps=3):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    _, kk, n, x, w, ws = qkv
    qa, sa = ops.bf16_int8_convrot_quantize(x, GROUP)
    qz, wz = torch.zeros_like(qa), torch.zeros_like(w)
    out = {}
    ms_r = timed(lambda: ops.int8_linear(qa, w, sa, ws, None))
    ms_z = timed(lambda: ops.int8_linear(qz, wz, sa, ws, None))
    out["int8_gemm_qkv"] = {"ms_bench_data": ms_r, "ms_zero_operands": ms_z, "ratio": ms_r / ms_z}
    del qa, qz, wz
    mean = sage_quant.key_channel_mean(k, "HND")
    q8, qs = sage_quant.quantize_per_block(q, BLK, "HND")
    k8, ks = sage_quant.quantize_per_block(k, BLK, "HND", mean)
    vt, _ = sage_quant.value_transpose(v, "HND")
    kw = dict(tensor_layout="HND", sm_scale=ATTN["d"] ** -0.5, blkq=BLK, blkk=BLK)
    ms_r = timed(lambda: attention_from_vt(q8, qs, k8, ks, vt, **kw))
    q8z, k8z, vtz = torch.zeros_like(q8), torch.zeros_like(k8), torch.zeros_like(vt)
    ms_z = timed(lambda: attention_from_vt(q8z, qs, k8z, ks, vtz, **kw))
    out["sage_attn"] = {"ms_bench_data": ms_r, "ms_zero_operands": ms_z, "ratio": ms_r / ms_z}
    return out


def extra_kernels(torch, dev, ops, lin, q, k, v, copy_gbs) -> dict:
    """Kernels of the path's next rows, timed outside the headline step (the
    metric's workload is the four linears and the attention): configs 1 and 2
    (the Wan-1.3B linear and attention shapes), the GELU-fused
    ConvRot quantizer at FFN-down (K13824), the fused Q/K RMSNorm + RoPE +
    INT8 producer at the attention shape (row-scope RMSNorm, interleaved
    full-width RoPE, as in a Wan block), and the dense W8A8 attention variant
    (INT8 PV) with its rotated Q/K and channel-wise V quantizers."""
    from comfyui_turing_utils_kernel.turing_sage import core as sage_core, quant as sage_quant
    from comfyui_turing_utils_kernel.turing_sage.custom_ops import qk_rms_rope_int8
    from tests import inputs

    def timed(fn, reps=10, batches=5):
        # the median over batches of back-to-back calls: these kernels run
        # between the step's power-limited ones, and single batches vary
        fn()
        torch.cuda.synchronize()
        per = []
        for _ in range(batches):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                fn()
            e1.record()
            torch.cuda.synchronize()
            per.append(e0.elapsed_time(e1) / reps)
        return sorted(per)[len(per) // 2]

    out = {}
    # config 1: the Wan-1.3B FFN-up linear, 4096 x 1536 -> 8960 with bias
    # (seed 0), its quantizer and GEMM timed separately
    xc = inputs.activation(4096, 1536, 0).to(dev)
    wc, wsc, bc = (t.to(dev) for t in inputs.weights(8960, 1536, 0))
    qc, sc = ops.bf16_int8_convrot_quantize(xc, GROUP)
    ms_q = timed(lambda: ops.bf16_int8_convrot_quantize(xc, GROUP), reps=50)
    ms_g = timed(lambda: ops.int8_linear(qc, wc, sc, wsc, bc), reps=50)
    flops = 2.0 * 4096 * 8960 * 1536
    nbytes = 3.0 * xc.numel() + 4.0 * xc.shape[0]
    out["c1_int8_gemm"] = {"ms_avg": ms_g, "tops": flops / ms_g / 1e9,
                           "frac_int8_peak": flops / ms_g / 1e9 / PEAK_INT8_TOPS, "shape": [4096, 1536, 8960],
                           "bias": True}
    out["c1_convrot_quant"] = {"ms_avg": ms_q, "gbs": nbytes / ms_q / 1e6, "frac_copy": nbytes / ms_q / 1e6 / copy_gbs}
    del xc, wc, wsc, bc, qc, sc
    # config 2: Sage attention at B1 H12 L8190 D128 (seed 1), the kernel alone
    # on prequantized Q/K and V^T; the planner's key split (kv_splits=None)
    # and the unsplit kernel
    from comfyui_turing_utils_kernel.turing_sage.core import attention_from_vt

    q2, k2, v2 = (t.to(dev) for t in inputs.attention(1, 12, 8190, 128, 1))
    st2 = sage_core.prequantize_sageattn(q2, k2, v2, "HND", BLKQ=BLK, BLKK=BLK)
    a2 = (st2.query_int8, st2.query_scale, st2.key_int8, st2.key_scale, st2.value_t)
    kw2 = dict(tensor_layout="HND", sm_scale=128 ** -0.5, blkq=BLK, blkk=BLK)
    flops = 4.0 * 12 * 8190 * 8190 * 128
    for tag, splits in (("c2_sage_attn", None), ("c2_sage_attn_unsplit", 1)):
        ms = timed(lambda: attention_from_vt(*a2, **kw2, kv_splits=splits), reps=50)
        out[tag] = {"ms_avg": ms, "tops": flops / ms / 1e9, "frac_int8_peak": flops / ms / 1e9 / PEAK_INT8_TOPS,
                    "shape": [1, 12, 8190, 128]}
    del q2, k2, v2, st2, a2
    x = next(t[3] for t in lin if t[1] == 13824)
    ms = timed(lambda: ops.bf16_gelu_int8_convrot_quantize(x, GROUP))
    nbytes = 3.0 * x.numel() + 4.0 * x.shape[0]
    out["gelu_convrot_quant_k13824"] = {"ms_avg": ms, "gbs": nbytes / ms / 1e6,
                                        "frac_copy": nbytes / ms / 1e6 / copy_gbs}
    b, h, l, d = q.shape
    g = torch.Generator().manual_seed(31)
    w = (1 + 0.1 * torch.randn(h * d, generator=g)).to(torch.bfloat16).to(dev)
    theta = torch.rand((1, l, 1, d // 2), generator=g) * 6.28
    freqs = torch.stack([torch.stack([theta.cos(), -theta.sin()], -1),
                         torch.stack([theta.sin(), theta.cos()], -1)], -2).to(torch.bfloat16).to(dev)
    ms = timed(lambda: qk_rms_rope_int8(q, k, w, w, freqs, 1e-6, d, "HND", "row", False, False, False))
    # Q and K: 2 B read + 1 B write per element (the row-scope pre-pass reads
    # them once more: 2 B per element, not counted as algorithmic work)
    nbytes = 2 * 3.0 * q.numel()
    out["qk_rms_rope_int8"] = {"ms_avg": ms, "gbs": nbytes / ms / 1e6, "frac_copy": nbytes / ms / 1e6 / copy_gbs,
                               "shape": [b, h, l, d], "norm_scope": "row", "rot_dim": d}
    state = sage_core.prequantize_w8a8attn(q, k, v)
    ms = timed(lambda: sage_core.w8a8attn_from_prequantized(state))
    flops = 4.0 * b * h * l * l * d
    out["w8a8_attn"] = {"ms_avg": ms, "tops": flops / ms / 1e9, "frac_int8_peak": flops / ms / 1e9 / PEAK_INT8_TOPS,
                        "shape": [b, h, l, d]}
    ms = timed(lambda: sage_quant.per_warp_int8_hadamard(q, k))
    out["w8a8_quant_qk"] = {"ms_avg": ms, "gbs": 2 * 3.0 * q.numel() / ms / 1e6}
    ms = timed(lambda: sage_quant.quantize_v_int8(v))
    # V read twice (amax pass, code pass), codes written once
    out["w8a8_quant_v"] = {"ms_avg": ms, "gbs": 5.0 * v.numel() / ms / 1e6}
    del state
    # the block's norm1 / norm2: LayerNorm + AdaLN over [1, L, H * D] with one
    # modulation row; 2 B read + 2 B written per element
    gen = torch.Generator(device=dev).manual_seed(37)
    xn = torch.randn(b, l, h * d, generator=gen, device=dev).to(torch.bfloat16)
    mod = (0.1 * torch.randn(b, 1, h * d, generator=gen, device=dev)).to(torch.bfloat16)
    ms = timed(lambda: ops.layer_norm_adaln(xn, mod, mod, 1e-6))
    nbytes = 4.0 * xn.numel()
    out["layer_norm_adaln"] = {"ms_avg": ms, "gbs": nbytes / ms / 1e6, "frac_copy": nbytes / ms / 1e6 / copy_gbs,
                               "frac_hbm_peak": nbytes / ms / 1e6 / PEAK_HBM_GBS, "shape": [b, l, h * d]}
    # the same norm fused with the next projection's ConvRot quantizer (G 128):
    # 2 B read + 1 B code written per element, a 4-byte scale per row; and
    # the two kernels it replaces
    ms = timed(lambda: ops.layer_norm_adaln_int8_convrot_quantize(xn, mod, mod, 1e-6, GROUP))
    ms_two = timed(lambda: ops.bf16_int8_convrot_quantize(
        ops.layer_norm_adaln(xn, mod, mod, 1e-6).view(b * l, h * d), GROUP))
    nbytes = 3.0 * xn.numel() + 4.0 * b * l
    out["layer_norm_adaln_convrot_quant"] = {"ms_avg": ms, "gbs": nbytes / ms / 1e6, "ms_two_kernels": ms_two,
                                             "shape": [b, l, h * d]}
    del xn, mod
    # C5: the whole Wan-14B block forward (norms, seven W8A8 projections, fused
    # Q/K producers, self- and cross-attention, gated residuals)
    from comfyui_turing_utils_kernel import wan_block

    cfg = wan_block.WanBlockConfig()
    block, text = wan_block.random_block(cfg, seed=4, device=dev)
    bx, be, bctx, bfreqs = wan_block.c5_inputs(text, dev)
    ms = timed(lambda: block(bx, be, bctx, bfreqs), reps=5)
    ops_ = wan_block.block_ops(cfg, bx.shape[1], bctx.shape[1])
    out["wan_block_c5"] = {"ms_avg": ms, "tops": ops_ / ms / 1e9, "frac_int8_peak": ops_ / ms / 1e9 / PEAK_INT8_TOPS,
                           "tokens": bx.shape[1], "text_tokens": bctx.shape[1]}
    del block, text, bx, be, bctx, bfreqs
    return out


def copy_bandwidth(torch, dev) -> float:
    """Achievable HBM bandwidth on this GPU: GB/s of a 1 GiB read + 1 GiB write
    elementwise kernel (median of 5, HIP events), outside the timed region."""
    src = torch.ones(1 << 28, dtype=torch.int32, device=dev)
    dst = torch.empty_like(src)
    times = []
    for _ in range(6):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        torch.neg(src, out=dst)
        b.record()
        b.synchronize()
        times.append(a.elapsed_time(b))
    del src, dst
    return 2.0 * (1 << 30) / (sorted(times[1:])[2] * 1e-3) / 1e9


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")
MFMA_FILE = os.path.join(ROOT, "profiles", "mfma_counters.json")
CSRC_DIR = os.path.join(ROOT, "comfyui-turing-utils_amd", "csrc")


# The sources each bench kernel is built from (the headers every kernel
# includes are added by kernel_sources_digest).
KERNEL_SOURCES = (
    ("convrot_quant", ("convrot_quant.hip", "ln_common.h")),
    ("int8_gemm", ("int8_gemm.hip",)),
    ("sage_kmean", ("sage_quant.hip",)),
    ("sage_quant", ("sage_quant.hip",)),
    ("sage_v_prep", ("sage_attn.hip", "attn_common.h")),
    ("sage_attn", ("sage_attn.hip", "attn_common.h")),
)


def kernel_sources_digest(kernel: str) -> str:
    """sha256 (first 16 hex digits) over the HIP sources and headers ``kernel``
    (a bench kernel name) is built from, in name order: the version stamp
    each entry of the committed counter files carries."""
    import hashlib

    files = next(f for prefix, f in KERNEL_SOURCES if kernel.startswith(prefix))
    h = hashlib.sha256()
    for name in sorted(files + ("tu_common.h",)) + ["../../include/tu_hip.h"]:
        with open(os.path.join(CSRC_DIR, name), "rb") as f:
            h.update(os.path.basename(name).encode() + b"\0" + f.read())
    return h.hexdigest()[:16]


def counters_source(path: str, kernel: str) -> dict:
    """Where the roofline's committed counter figures for ``kernel`` come
    from, and whether they were captured from the kernel's sources in this
    tree."""
    try:
        with open(path) as f:
            stamp = (json.load(f).get(kernel) or {}).get("_kernel_sources")
    except (OSError, ValueError):
        stamp = None
    return {"file": os.path.relpath(path, ROOT), "kernel_sources": stamp,
            "current": stamp is not None and stamp == kernel_sources_digest(kernel)}


def measured_mfma(kernel: str):
    """MFMA busy fraction and clock of ``kernel`` at this workload, from the
    committed rocprofv3 --pmc passes (SQ_VALU_MFMA_BUSY_CYCLES over the SIMD
    cycles; GRBM_GUI_ACTIVE over the kernel time), or None when not committed."""
    try:
        with open(MFMA_FILE) as f:
            return json.load(f).get(kernel)
    except (OSError, ValueError):
        return None


def measured_traffic(kernel: str):
    """Bytes per launch of ``kernel`` that its L2 requested from the fabric at
    this workload (read + write requests times their sizes, from the committed
    rocprofv3 --pmc passes), or None when no such measurement is committed."""
    try:
        with open(TRAFFIC_FILE) as f:
            entry = json.load(f).get(kernel)
    except (OSError, ValueError):
        return None
    return None if entry is None else float(entry["bytes_per_launch"])


def cpu_baseline(budget_s: float):
    """CPU baseline on a bounded sample of the same workload, on this host's cores.

    ``value`` is the reference's CPU path, its PyTorch fallback (the
    "dequantized matmul / SDPA" of the metric's definition): the ffn-up linear
    (K=5120, N=13824) as ``torch.nn.functional.linear`` in bf16 on the
    dequantized weight ``bf16(W * w_scale)`` (prepared outside the timing), on
    a sample of rows, and Sage attention's fallback
    ``scaled_dot_product_attention`` in bf16 on a sample of query rows of one
    head of config 3 against all 32760 keys.  Each is timed as the median of
    three calls; the two rates are combined with the GPU step's op mix into
    one step-equivalent rate.  ``oracle`` times the CPU oracle (oracle/, the
    plain-C restatement of the reference arithmetic: ConvRot quantize + exact
    INT8 GEMM + epilogue; K mean, INT8 Q/K, softmax with bf16 P) on the same
    kind of sample.  Sample sizes are calibrated so the whole baseline takes
    about ``budget_s`` seconds.
    """
    import numpy as np
    import torch

    from oracle import oracle
    from tests import inputs

    threads = oracle.num_threads()
    k, n = 5120, 13824
    x_all = inputs.activation(4096, k, 5)
    w, ws, _ = inputs.weights(n, k, 5, with_bias=False)
    wn, wsn = w.numpy(), ws.numpy()
    lin_ops = sum(2.0 * M_TOKENS * nn * kk_ for _, kk_, nn in LINEARS)
    l, d = ATTN["l"], ATTN["d"]
    attn_ops = 4.0 * ATTN["b"] * ATTN["h"] * l ** 2 * d
    q, kk, v = inputs.attention(1, 1, l, d, 2)

    def median_time(fn, reps=3):
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return sorted(ts)[reps // 2]

    # ---- the reference's PyTorch CPU fallback (the headline value)
    wd = (w.float() * ws[:, None]).to(torch.bfloat16)
    torch.nn.functional.linear(x_all[:64], wd)  # warm-up
    probe = median_time(lambda: torch.nn.functional.linear(x_all[:256], wd), 1)
    rows_t = int(min(4096, max(256, 0.12 * budget_s / probe * 256)))
    xs = x_all[:rows_t]
    t_tl = median_time(lambda: torch.nn.functional.linear(xs, wd))
    tl_tops = 2.0 * rows_t * n * k / t_tl / 1e12
    sdpa = torch.nn.functional.scaled_dot_product_attention
    sdpa(q[:, :, :64], kk, v)  # warm-up
    probe = median_time(lambda: sdpa(q[:, :, :256], kk, v), 1)
    rows_ta = int(min(l, max(256, 0.12 * budget_s / probe * 256)))
    qs_ = q[:, :, :rows_ta]
    t_ta = median_time(lambda: sdpa(qs_, kk, v))
    ta_tops = 4.0 * rows_ta * l * d / t_ta / 1e12
    torch_step = lin_ops / (tl_tops * 1e12) + attn_ops / (ta_tops * 1e12)

    # ---- the CPU oracle on the same kind of sample
    def oracle_linear(rows):
        t0 = time.perf_counter()
        qa, sa = oracle.convrot_quant(inputs.bits(x_all[:rows]), GROUP)
        oracle.epilogue_bf16(oracle.int8_gemm_i32(qa, wn), sa, wsn)
        return time.perf_counter() - t0

    probe = oracle_linear(16)
    rows = int(min(4096, max(16, 0.25 * budget_s / probe * 16)))
    t_lin = oracle_linear(rows)
    lin_tops = 2.0 * rows * n * k / t_lin / 1e12
    qb, kb, vb = inputs.bits(q), inputs.bits(kk), inputs.bits(v)

    def oracle_attention(nrows):
        t0 = time.perf_counter()
        mean = oracle.sage_kmean(kb)
        k8, ks = oracle.sage_quant(kb, BLK, mean)
        q8, qs = oracle.sage_quant(qb[:, :, :nrows], BLK)
        sel = np.stack([np.zeros(nrows, np.int64), np.zeros(nrows, np.int64), np.arange(nrows)], 1)
        oracle.sage_attn_rows(q8, qs, BLK, k8, ks, BLK, vb, d ** -0.5, sel)
        return time.perf_counter() - t0

    probe = oracle_attention(threads)
    rows_a = int(min(l, max(threads, 0.25 * budget_s / probe * threads)))
    t_att = oracle_attention(rows_a)
    att_tops = 4.0 * rows_a * l * d / t_att / 1e12
    step_s = lin_ops / (lin_tops * 1e12) + attn_ops / (att_tops * 1e12)

    cpu_model = ""
    try:
        with open("/proc/cpuinfo") as f:
            cpu_model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), "")
    except OSError:
        pass
    return {
        "value": (lin_ops + attn_ops) / torch_step / 1e12,
        "unit": "TOPS",
        "cores": torch.get_num_threads(),
        "kind": "reference",
        "path": "the reference's PyTorch CPU fallback (torch bf16 linear on the dequantized weight; torch bf16 SDPA), "
                "run through this host's torch; not a build of the reference's CUDA sources",
        "cpu_model": cpu_model,
        "host_cpu_count": os.cpu_count(),
        "sample": f"ffn-up bf16 linear on the dequantized weight, {rows_t} of 32760 rows ({t_tl:.2f} s, "
                  f"{tl_tops:.3f} TFLOP/s), and bf16 SDPA on {rows_ta} query rows x 32760 keys of one head "
                  f"({t_ta:.2f} s, {ta_tops:.3f} TFLOP/s), medians of 3, combined with the step's op mix; "
                  f"projected step {torch_step:.1f} s",
        "oracle": {
            "value": (lin_ops + attn_ops) / step_s / 1e12,
            "unit": "TOPS",
            "cores": threads,
            "kind": "port",
            "sample": f"CPU oracle: ffn-up ConvRot W8A8 linear on {rows} of 32760 rows ({t_lin:.2f} s, "
                      f"{lin_tops:.4f} TOPS) and Sage attention on {rows_a} query rows x 32760 keys of one head "
                      f"({t_att:.2f} s, {att_tops:.4f} TOPS), combined with the step's op mix; "
                      f"projected step {step_s:.0f} s",
        },
    }

if __name__ == "__main__":
    sys.exit(main())
