"""Hardware and model constants for the MI355X build.

Peaks are AMD's published MI355X figures (AMD Instinct MI355X product page and CDNA 4 white
paper): 8.0 TB/s HBM3E, 288 GB, 256 CUs in 8 XCDs, 256 MB Infinity Cache (MALL), dense (no
sparsity) matrix throughput 2.5 PFLOP/s fp16/bf16, 5.0 fp8. The reference keeps the same kind of
table for its NVIDIA targets (kernels/config.py:13-28 of the reference).
"""

from __future__ import annotations

GPU_SPECS = {
    "MI355X": {
        "peak_gbps": 8000.0,
        "peak_fp16_tflops": 2500.0,
        "peak_fp8_tflops": 5000.0,
        "peak_fp32_vector_tflops": 157.3,
        "hbm_gb": 288,
        "cus": 256,
        "xcds": 8,
        "mall_mb": 256,
        "l2_mb_per_xcd": 4,
        "source": "https://www.amd.com/en/products/accelerators/instinct/mi350/mi355x.html",
    },
}
PEAK_GBPS = GPU_SPECS["MI355X"]["peak_gbps"]

MODEL_ID = "Qwen/Qwen2.5-1.5B-Instruct"  # architecture only: weights are random-init here
GROUP_SIZE = 128

# W4A16 benchmark layers (label, N, K): Qwen2.5-1.5B with fused qkv and gate_up, as the
# reference's W4_SHAPES (kernels/config.py:71-74), plus the separate q/k/v/o shapes of the
# MI355X configs.
W4_SHAPES = [
    ("qwen_qkv", 2048, 1536), ("qwen_o", 1536, 1536), ("qwen_gate_up", 17920, 1536),
    ("qwen_down", 1536, 8960), ("8b_up", 14336, 4096), ("8b_down", 4096, 14336),
]
QWEN_SHAPES = [
    ("q", 1536, 1536), ("k", 256, 1536), ("v", 256, 1536), ("o", 1536, 1536),
    ("gate_up", 17920, 1536), ("down", 1536, 8960),
]

# Qwen2.5-1.5B architecture (config 4).
QWEN25_15B = dict(
    vocab_size=151936, hidden_size=1536, intermediate_size=8960, num_hidden_layers=28,
    num_attention_heads=12, num_key_value_heads=2, head_dim=128, rope_theta=1_000_000.0,
    rms_norm_eps=1e-6, tie_word_embeddings=True,
)
