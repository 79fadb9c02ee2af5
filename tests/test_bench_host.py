"""Host logic of bench.py that needs no GPU: the per-kernel source stamps
that decide whether the committed rocprofv3 counter files still describe the
kernels in this tree."""
from __future__ import annotations

import json

import bench

BENCH_KERNELS = ("convrot_quant_k5120", "convrot_quant_k13824", "int8_gemm_qkv", "int8_gemm_out",
                 "int8_gemm_ffn_up", "int8_gemm_ffn_down", "sage_kmean", "sage_quant_q", "sage_quant_k",
                 "sage_v_prep", "sage_attn")


def test_every_bench_kernel_has_a_source_stamp():
    for name in BENCH_KERNELS:
        digest = bench.kernel_sources_digest(name)
        assert len(digest) == 16 and int(digest, 16) >= 0
    # kernels built from different sources get different stamps, kernels of
    # one source file the same
    assert bench.kernel_sources_digest("sage_attn") != bench.kernel_sources_digest("int8_gemm_qkv")
    assert bench.kernel_sources_digest("int8_gemm_qkv") == bench.kernel_sources_digest("int8_gemm_ffn_down")
    assert bench.kernel_sources_digest("sage_quant_q") == bench.kernel_sources_digest("sage_kmean")


def test_counters_source_is_current_only_for_a_matching_stamp(tmp_path):
    path = tmp_path / "counters.json"
    path.write_text(json.dumps({
        "sage_attn": {"_kernel_sources": bench.kernel_sources_digest("sage_attn"), "mfma_busy": 0.6},
        "int8_gemm_qkv": {"_kernel_sources": "0" * 16, "mfma_busy": 0.6},
    }))
    assert bench.counters_source(str(path), "sage_attn")["current"]
    assert not bench.counters_source(str(path), "int8_gemm_qkv")["current"]
    assert not bench.counters_source(str(path), "sage_kmean")["current"]  # no entry for it
    assert not bench.counters_source(str(tmp_path / "missing.json"), "sage_attn")["current"]
