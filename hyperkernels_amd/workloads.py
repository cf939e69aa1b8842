"""The benchmark configurations this kernel surface is measured on, and their work accounting.

Byte and FLOP conventions follow the reference's published numbers (back-derived from its
README latency x throughput, README.md:186-199): attention fwd FLOP = 4 B H T^2 d (halved when
causal), bwd = 2.5x fwd; LN fwd bytes = 2 N C sizeof(T), bwd = 3 N C sizeof(T);
GELU fwd = 2 n sizeof(T), bwd = 3 n sizeof(T); CE fwd = R V 4, bwd = 2 R V 4; reduce = R V 4; AdamW = 7 P 4;
GEMM = 2 M N K per batch.
"""
from __future__ import annotations

# GPT-2 small (124M): the 148 fp32 parameter tensors the AdamW configuration steps over.
GPT2_VOCAB, GPT2_CTX, GPT2_C, GPT2_LAYERS = 50257, 1024, 768, 12


def gpt2_param_shapes() -> list[tuple[int, ...]]:
    C = GPT2_C
    shapes: list[tuple[int, ...]] = [(GPT2_VOCAB, C), (GPT2_CTX, C)]
    for _ in range(GPT2_LAYERS):
        shapes += [(C,), (C,), (C, 3 * C), (3 * C,), (C, C), (C,), (C,), (C,), (C, 4 * C),
                   (4 * C,), (4 * C, C), (C,)]
    shapes += [(C,), (C,)]
    return shapes


def numel(shape) -> int:
    n = 1
    for s in shape:
        n *= s
    return n


GPT2_NUM_PARAMS = sum(numel(s) for s in gpt2_param_shapes())
assert len(gpt2_param_shapes()) == 148 and GPT2_NUM_PARAMS == 124_439_808

# BASELINE.json configs (their index in `configs`).
LN = dict(rows=4096, cols=768, eps=1e-5)                       # configs[0]
GELU = dict(shape=(8, 1024, 3072))                             # configs[1]
CE = dict(rows=8192, vocab=50257)                              # configs[1]
ADAMW = dict(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1)  # configs[1]
ATTN = dict(B=8, H=12, T=1024, d=64)                           # configs[2], configs[3]
BGEMM = dict(M=8192, K=1280, N=5120)                           # configs[4]
SGEMM = dict(M=4096, N=4096, K=4096, split_k=4)                # configs[4]


def ln_fwd_bytes(rows, cols, esize=4):
    return 2 * rows * cols * esize


def ln_bwd_bytes(rows, cols, esize=4):
    return 3 * rows * cols * esize


def gelu_fwd_bytes(n, esize):
    return 2 * n * esize


def gelu_bwd_bytes(n, esize):
    return 3 * n * esize


def ce_fwd_bytes(rows, vocab):
    return rows * vocab * 4


def ce_bwd_bytes(rows, vocab):
    return 2 * rows * vocab * 4


def adamw_bytes(params):
    return 7 * params * 4


def attn_fwd_flop(B, H, T, d, causal):
    f = 4 * B * H * T * T * d
    return f // 2 if causal else f


def attn_bwd_flop(B, H, T, d, causal):
    return 5 * attn_fwd_flop(B, H, T, d, causal) // 2


def gemm_flop(M, N, K, batch=1):
    return 2 * M * N * K * batch


# MI355X published peaks (AMD): HBM3E bandwidth and dense matrix throughput.
PEAK_HBM_GBS = 8000.0
PEAK_TFLOPS = {"bf16": 2516.6, "fp32_matrix": 157.3,
               # fp32 products computed as a bf16x3 split: three bf16 MFMA products each
               "bf16x3": 2516.6 / 3}
