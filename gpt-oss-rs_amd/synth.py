"""Seeded synthetic inputs for the MoE block at the benchmark configurations.

Shapes and distributions of the GPT-OSS-20B MoE layer: hidden rows
bf16(N(0,1)) RMS-normalised and rounded to bf16, router weights bf16
N(0, 0.02) with a bf16 bias, expert biases bf16 N(0, 0.02), and MXFP4 expert
tensors generated on the device (uniform codes, E8M0 exponents -8..-4; see
gossmx_weights_generate). Router logits for the decode configuration can be
injected so that expert popularity follows a Zipf law.
"""
from __future__ import annotations

import numpy as np

HIDDEN = 2880
INTERMEDIATE = 2880
EXPERTS_20B = 32
EXPERTS_120B = 128
TOP_K = 4
LAYERS_20B = 24
LAYERS_120B = 36


def bf16_bits(a: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even (NaN quieted)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    up = ((u & 0x8000) != 0) & ((u & 0x17FFF) != 0)
    hi = np.where(nan, (u >> 16) | 0x40, (u >> 16) + up.astype(np.uint64))
    return (hi & 0xFFFF).astype(np.uint16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def hidden_rows(rng: np.random.Generator, m: int, h: int = HIDDEN, normalise: bool = True) -> np.ndarray:
    x = bf16_to_f32(bf16_bits(rng.standard_normal((m, h)).astype(np.float32)))
    if normalise:
        ss = np.einsum("ij,ij->i", x.astype(np.float64), x.astype(np.float64)) / h
        x = (x / np.sqrt(ss + 1e-5)[:, None]).astype(np.float32)
    return bf16_bits(x)


def normal_bf16(rng: np.random.Generator, shape, std: float) -> np.ndarray:
    return bf16_bits((rng.standard_normal(shape) * std).astype(np.float32))


def dense_layer_params(rng: np.random.Generator, experts: int = EXPERTS_20B, hidden: int = HIDDEN,
                       intermediate: int = INTERMEDIATE) -> dict:
    """Router weight/bias and expert biases of one layer (f32 biases hold bf16 values)."""
    return {
        "router_weight": normal_bf16(rng, (experts, hidden), 0.02),
        "router_bias": bf16_to_f32(normal_bf16(rng, experts, 0.02)),
        "gate_up_bias": bf16_to_f32(normal_bf16(rng, experts * 2 * intermediate, 0.02)),
        "down_bias": bf16_to_f32(normal_bf16(rng, experts * hidden, 0.02)),
    }


def zipf_logits(rng: np.random.Generator, m: int, experts: int, top_k: int = TOP_K, s: float = 1.1) -> np.ndarray:
    """Logits [m][experts] (bf16 values) whose top-k sets follow Zipf(s)
    popularity over a random expert permutation, top_k distinct experts per row."""
    perm = rng.permutation(experts)
    p = 1.0 / np.arange(1, experts + 1, dtype=np.float64) ** s
    p = p / p.sum()
    popularity = np.empty(experts)
    popularity[perm] = p
    logits = np.clip(rng.standard_normal((m, experts)), -3.0, 1.5).astype(np.float32)
    for r in range(m):
        chosen = rng.choice(experts, size=top_k, replace=False, p=popularity)
        logits[r, chosen] = 2.0 + np.sort(rng.uniform(0.0, 2.0, top_k))[::-1]
    return bf16_to_f32(bf16_bits(logits))


def uniform_logits(rng: np.random.Generator, m: int, experts: int) -> np.ndarray:
    """Near-uniform routing: i.i.d. logits, bf16 values."""
    return bf16_to_f32(bf16_bits(rng.standard_normal((m, experts)).astype(np.float32)))


def model_weights(config: dict, normal) -> dict:
    """Dense tensors of a random-init GPT-OSS model (config: the gossmx_model_config
    fields): embedding, lm_head and the q/k/v/o matrices bf16 N(0, 0.02); their
    biases and the attention sinks N(0, 0.02) and the RMSNorm weights N(1, 0.02),
    as f32 holding bf16 values. Layer i is sliding when i is even (GPT-OSS's
    alternating layer_types). normal(n, std) returns n bf16 bit patterns."""
    V, H = config["vocab"], config["hidden"]
    QW, KW = config["heads"] * config["head_dim"], config["kv_heads"] * config["head_dim"]

    def vec(n, mean=0.0):
        return (bf16_to_f32(normal(n, 0.02)) + np.float32(mean)).astype(np.float32)

    layers = []
    for i in range(config["layers"]):
        layers.append({
            "input_norm": bf16_to_f32(bf16_bits(vec(H, 1.0))), "post_attention_norm": bf16_to_f32(bf16_bits(vec(H, 1.0))),
            "q_weight": normal(QW * H, 0.02).reshape(QW, H), "q_bias": vec(QW),
            "k_weight": normal(KW * H, 0.02).reshape(KW, H), "k_bias": vec(KW),
            "v_weight": normal(KW * H, 0.02).reshape(KW, H), "v_bias": vec(KW),
            "o_weight": normal(H * QW, 0.02).reshape(H, QW), "o_bias": vec(H),
            "sinks": vec(config["heads"]), "sliding": i % 2 == 0,
        })
    return {"embedding": normal(V * H, 0.02).reshape(V, H), "lm_head": normal(V * H, 0.02).reshape(V, H),
            "final_norm": bf16_to_f32(bf16_bits(vec(H, 1.0))), "layers": layers}


def numpy_normal(rng: np.random.Generator):
    """normal(n, std) for model_weights from a numpy generator (small models)."""
    return lambda n, std: bf16_bits(rng.standard_normal(n, dtype=np.float32) * np.float32(std))
