"""The synthetic Qwen3-30B-A3B MoE workloads (shapes, seeds, router bias).

Weights: experts and routers ~ N(0, 0.02) from include/mia/synth.h with
WEIGHT_SEED, experts quantized to Q8_0, ffn_norm = 1, eps = 1e-6,
renormalised top-8 of 128. Inputs: x ~ N(0, 1) with X_SEED.
"""
import numpy as np

WEIGHT_SEED = 42
X_SEED = 43
SHAPE = dict(dim=2048, n_experts=128, n_active=8, expert_hidden=768, norm_topk=1,
             norm_eps=1e-6)

# name -> (layers, tokens, skewed router)
WORKLOADS = {
    "decode1": dict(layers=1, tokens=1, skew=False,
                    doc="single MoE layer, decode batch 1"),
    "prefill512": dict(layers=1, tokens=512, skew=False,
                       doc="single MoE layer, prefill T=512"),
    "skew2048": dict(layers=1, tokens=2048, skew=True,
                     doc="single MoE layer, T=2048, Zipf(1.2)-biased router"),
    "decode48": dict(layers=48, tokens=1, skew=False,
                     doc="48-layer MoE-only stack, decode batch 1"),
    "batch64x48": dict(layers=48, tokens=64, skew=False,
                       doc="48-layer MoE-only stack, 64 independent sequences"),
    "prefill4096": dict(layers=1, tokens=4096, skew=False,
                        doc="single MoE layer, prefill T=4096"),
    "prefill4096x48": dict(layers=48, tokens=4096, skew=False,
                           doc="48-layer MoE-only stack, prefill T=4096"),
}

# Zipf exponent and the strength that gives, at T=2048, ~40 % of the
# assignments to the top 4 experts and ~30 experts none.
ZIPF_S = 1.2
ZIPF_BETA = 0.95
ZIPF_SEED = 7

_M64 = (1 << 64) - 1


def _mix(z):
    z ^= z >> 30
    z = (z * 0xBF58476D1CE4E5B9) & _M64
    z ^= z >> 27
    z = (z * 0x94D049BB133111EB) & _M64
    z ^= z >> 31
    return z


def zipf_ranks(n_experts, seed=ZIPF_SEED):
    """A seeded permutation: rank (0 = most favoured) of each expert."""
    keys = [_mix((seed * 0x9E3779B97F4A7C15 + e + 1) & _M64) for e in range(n_experts)]
    order = sorted(range(n_experts), key=lambda e: keys[e])
    ranks = np.zeros(n_experts, dtype=np.int64)
    for r, e in enumerate(order):
        ranks[e] = r
    return ranks


def zipf_bias(n_experts=128, s=ZIPF_S, beta=ZIPF_BETA, seed=ZIPF_SEED):
    """bias_e = -beta * s * ln(rank_e + 1): a Zipf(s) prior on the router
    logits, added after the router product and before the softmax."""
    ranks = zipf_ranks(n_experts, seed)
    return (-beta * s * np.log(ranks + 1.0)).astype(np.float32)


def bytes_per_step(layers, tokens, n_touched_per_layer, shape=SHAPE):
    """Algorithmic HBM bytes of one pass: each touched expert's Q8_0 blob
    (36-byte blocks) once, the fp32 router once, x read and written once
    per layer."""
    d, eh = shape["dim"], shape["expert_hidden"]
    blob = 3 * eh * d // 32 * 36
    router = shape["n_experts"] * d * 4
    return sum(n * blob + router + tokens * d * 4 * 2 for n in n_touched_per_layer)


def ops_per_step(layers, tokens, shape=SHAPE):
    """Integer/float ops of one pass (2 per multiply-add): the K expert
    products (3 matrices) and the router per token and layer."""
    d, eh, K, E = shape["dim"], shape["expert_hidden"], shape["n_active"], shape["n_experts"]
    return layers * tokens * (K * 3 * eh * d * 2 + E * d * 2)
