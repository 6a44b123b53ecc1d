"""The benchmark configurations as data: shapes, block types and seeds.

Every input is drawn by the shared C generator (include/mynah_synth.h), so the
GPU path, the CPU oracle and the compiled reference see identical bytes.
Seed scheme (all derived from a config seed s, 0 for every configuration):
  * matrix i of a config:        blocks from substream(s, 2 i), x from substream(s, 2 i + 1)
  * Qwen3 model tensors:         mynah_synth_qwen3_fill(seed = s)
  * Qwen3 KV prefill, layer l:   K from substream(kv, 2 l), V from substream(kv, 2 l + 1),
                                 kv = substream(s, 1 << 20)
  * Qwen3 first decode token:    uniform over the vocabulary from substream(s, 1 << 21)
                                 (configs[4]'s prompt: the first 2048 values of that stream)
  * prefill activations (C4):    X from substream(s, 1 << 22 + i) for matrix i
  * teacher-forced decode inputs: uniform over the vocabulary from substream(s, 1 << 23)
"""
from __future__ import annotations

from dataclasses import dataclass

Q4_0, Q8_0, Q4_K, Q5_K, Q6_K = 2, 8, 12, 13, 14
TYPE_NAME = {Q4_0: "Q4_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K"}

# The adjacent block types (Q5_K, Q4_0): shapes of their parity cases —
# (type, rows, cols, token counts of the batched product). Ragged rows,
# Q4_0 rows that are not whole 256-value units, and token counts around the
# kernels' tiles (8 tokens per Q4_0 lane group, 64 per GEMM tile).
ADJACENT = ((Q5_K, 37, 512, (3, 9)), (Q5_K, 5, 2048, (2, 65)), (Q5_K, 130, 1024, (64,)),
            (Q4_0, 37, 96, (3, 9)), (Q4_0, 8, 4096, (2, 17)), (Q4_0, 3, 32, (8,)),
            (Q4_0, 70, 2080, (5, 64)))


@dataclass(frozen=True)
class Matrix:
    name: str
    qtype: int
    rows: int
    cols: int


# Q4_K ffn_down-shaped matvec of Qwen3-0.6B (1024 x 3072).
C1 = [Matrix("q4k_1024x3072", Q4_K, 1024, 3072)]

# Q6_K and Q8_0 at the Qwen3-0.6B projection shapes + the Q6_K head.
C2_SHAPES = [("q", 2048, 1024), ("kv", 1024, 1024), ("o", 1024, 2048), ("gate_up", 3072, 1024)]
C2 = ([Matrix(f"q6k_{n}_{r}x{c}", Q6_K, r, c) for n, r, c in C2_SHAPES]
      + [Matrix(f"q80_{n}_{r}x{c}", Q8_0, r, c) for n, r, c in C2_SHAPES]
      + [Matrix("q6k_head_151936x1024", Q6_K, 151936, 1024)])

# prefill GEMM at Qwen3-1.7B shapes, M = 512 tokens.
C4_TOKENS = 512
C4 = [Matrix("q4k_q_4096x2048", Q4_K, 4096, 2048),
      Matrix("q4k_kv_2048x2048", Q4_K, 2048, 2048),
      Matrix("q4k_o_2048x2048", Q4_K, 2048, 2048),
      Matrix("q4k_gate_6144x2048", Q4_K, 6144, 2048),
      Matrix("q4k_up_6144x2048", Q4_K, 6144, 2048),
      Matrix("q6k_down_2048x6144", Q6_K, 2048, 6144)]

# Qwen3-4B decode GEMV shapes (the >= 70 % of HBM target), Q4_K_M classes.
QWEN3_4B_GEMV = [Matrix("q4k_q_4096x2560", Q4_K, 4096, 2560),
                 Matrix("q4k_kv_1024x2560", Q4_K, 1024, 2560),
                 Matrix("q4k_o_2560x4096", Q4_K, 2560, 4096),
                 Matrix("q4k_gate_up_9728x2560", Q4_K, 9728, 2560),
                 Matrix("q4k_down_2560x9728", Q4_K, 2560, 9728),
                 Matrix("q6k_down_2560x9728", Q6_K, 2560, 9728),
                 Matrix("q6k_v_1024x2560", Q6_K, 1024, 2560),
                 Matrix("q6k_head_151936x2560", Q6_K, 151936, 2560)]


@dataclass(frozen=True)
class Qwen3Shape:
    n_layers: int
    d_model: int
    d_ff: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    vocab: int
    rms_eps: float = 1e-6
    rope_theta: float = 1e6


QWEN3_06B = Qwen3Shape(28, 1024, 3072, 16, 8, 128, 151936)
QWEN3_17B = Qwen3Shape(28, 2048, 6144, 16, 8, 128, 151936)
QWEN3_4B = Qwen3Shape(36, 2560, 9728, 32, 8, 128, 151936)
# A small model with the same structure, for quick CPU / GPU parity runs.
QWEN3_TINY = Qwen3Shape(3, 512, 768, 4, 2, 128, 4096)

C3_PREFILL = 512      # KV positions prefilled with N(0, 1)
C3_STEPS = 64         # greedy steps the token parity covers

C5_PROMPT = 2048      # prompt tokens, uniform over the vocabulary
C5_STEPS = 256        # greedy steps after the prompt
C5_GOLDEN_PROMPT = 8  # the prefix the compiled reference's golden run covers
C5_GOLDEN_STEPS = 8
# configs[4]'s decode at context 2048 on the CPU baseline: the 4B model with
# 2048 KV positions prefilled with N(0, 1) (the work of one step depends on
# the context length, not on the cached values), then greedy steps.
C5_CPU_KV = 2048
C5_CPU_STEPS = 10

MATRIX_SEED_STRIDE = 2
KV_SEED_INDEX = 1 << 20
TOKEN_SEED_INDEX = 1 << 21
PREFILL_X_INDEX = 1 << 22
FORCED_SEED_INDEX = 1 << 23

# Teacher-forced decode parity (configs[2]'s model and KV prefill): the input
# of every step is drawn uniformly instead of being the previous step's
# greedy id, so each step's logits (and greedy id) differ; the compiled
# reference's logits of every step are the golden vectors.
C3_FORCED_STEPS = 64
FORCED_SAMPLE_STRIDE = 293   # every 293rd logit of each step kept in full

# configs[4] end to end against the compiled reference: the greedy ids of
# all 256 steps and the top-64 logits of the steps listed here.
C5_SNAPSHOT_STEPS = (0, 1, 31, 63, 127, 191, 255)


def matrix_seeds(substream, config_seed: int, i: int) -> tuple[int, int]:
    """(weight seed, activation seed) of matrix i of a config."""
    return substream(config_seed, 2 * i), substream(config_seed, 2 * i + 1)


def kv_prefill(substream, normal, shape: Qwen3Shape, config_seed: int, n: int):
    """K and V prefill [layer][n][kv_dim] f32 of a decode config (N(0, 1));
    `normal(seed, count)` is the shared generator's f32 normal vector."""
    import numpy as np
    kv_seed = substream(config_seed, KV_SEED_INDEX)
    kvd = shape.n_kv_heads * shape.head_dim
    k = np.empty((shape.n_layers, n * kvd), np.float32)
    v = np.empty((shape.n_layers, n * kvd), np.float32)
    for layer in range(shape.n_layers):
        k[layer] = normal(substream(kv_seed, 2 * layer), n * kvd)
        v[layer] = normal(substream(kv_seed, 2 * layer + 1), n * kvd)
    return k, v


def c5_prompt(uniform, substream, vocab: int, n: int = C5_PROMPT, config_seed: int = 0):
    """configs[4]'s prompt: n ids uniform over the vocabulary (the stream whose
    first value is the decode configs' first token); `uniform(seed, n, bound)`
    is the shared generator's uniform vector."""
    return uniform(substream(config_seed, TOKEN_SEED_INDEX), n, vocab)


def forced_inputs(uniform, substream, vocab: int, n: int, config_seed: int = 0):
    """The inputs of a teacher-forced decode run: n ids uniform over the
    vocabulary."""
    return uniform(substream(config_seed, FORCED_SEED_INDEX), n, vocab)
