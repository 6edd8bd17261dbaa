"""The benchmark configurations and their synthetic-input definitions.

Shapes follow the five BASELINE configurations of the MoE teacher layer
(the reference's own teacher shape is 512 experts, top-10, width 640 with a
shared expert: src/qwen.c:11-37).  Every tensor comes from the counter-hash
generator (stream per tensor, key = seed, index = element), which is exact
integer + IEEE arithmetic, so the GPU fill kernel, the CPU oracle and any host
produce the same bits.
"""
import math

import numpy as np

# generator stream per tensor
STREAM_X = 1
STREAM_W_ROUTER = 2
STREAM_W_GATE_UP = 3
STREAM_W_DOWN = 4
STREAM_W_SH_GATE_UP = 5
STREAM_W_SH_DOWN = 6
STREAM_PERM = 7

STD_X = 1.0
STD_W = 0.02

CONFIGS = {
    1: dict(name="tiny", rows=256, d=512, experts=8, topk=2, inter=1024, shared=0, skew=False),
    2: dict(name="decode", rows=128, d=2048, experts=128, topk=8, inter=768, shared=0, skew=False),
    3: dict(name="prefill", rows=2048, d=2048, experts=128, topk=8, inter=768, shared=0, skew=False),
    4: dict(name="skewed", rows=2048, d=2048, experts=128, topk=8, inter=768, shared=0, skew=True),
    5: dict(name="fine_shared", rows=4096, d=2048, experts=512, topk=10, inter=512, shared=512, skew=False),
}

HEADLINE = 3

# The reference teacher's own MoE shape (src/qwen.c:11-37, src/qwen.h:20-21):
# hidden 2560, 512 experts, top-10, expert and shared width 640; rows = the
# repo's training batch of 8 x 256 tokens
TEACHER = dict(name="teacher", rows=2048, d=2560, experts=512, topk=10, inter=640, shared=640, skew=False)

# Config 3's shape with a mixed expert load: MIXED_HOT experts get a router
# bias of MIXED_BIAS, which puts each of them in about 70% of the tokens'
# top-8, so together they hold about 35% of the rows (~1400 each, hot) and
# the other 124 experts about 85 rows each (cold).  Neither tile's bucket
# holds every row: the per-call tile choice has to leave one bucket on the
# other bucket's tile.
MIXED_HOT = (3, 40, 77, 114)
MIXED_BIAS = 2.0
MIXED = dict(name="mixed", rows=2048, d=2048, experts=128, topk=8, inter=768, shared=0, skew="mixed")

_M64 = (1 << 64) - 1


def _mix64(x):
    x &= _M64
    a = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & _M64
    b = ((a ^ (a >> 27)) * 0x94D049BB133111EB) & _M64
    return b ^ (b >> 31)


def hash_u64(stream, key, i):
    """SplitMix64 finaliser applied to (stream, key, index) (src/hash.c:5-13)."""
    return _mix64(_mix64(_mix64(stream + 0x9E3779B97F4A7C15) ^ key) ^ i)


def skew_bias(experts, seed=0):
    """Per-expert router bias b_e = 3*log(1/rank_e^1.2) with rank a seeded
    permutation of 1..experts (Fisher-Yates driven by the counter hash)."""
    rank = list(range(1, experts + 1))
    for i in range(experts - 1, 0, -1):
        j = hash_u64(STREAM_PERM, seed, i) % (i + 1)
        rank[i], rank[j] = rank[j], rank[i]
    return np.array([3.0 * math.log(1.0 / (r ** 1.2)) for r in rank], dtype=np.float32)


def mixed_bias(experts):
    """Router bias of the MIXED workload: MIXED_BIAS on MIXED_HOT, 0 elsewhere."""
    b = np.zeros(experts, dtype=np.float32)
    b[[e for e in MIXED_HOT if e < experts]] = np.float32(MIXED_BIAS)
    return b


def router_bias(cfg, seed=0):
    """The router bias a configuration's inputs carry, or None."""
    if cfg.get("skew") == "mixed":
        return mixed_bias(cfg["experts"])
    if cfg.get("skew"):
        return skew_bias(cfg["experts"], seed)
    return None


def shape_of(cfg):
    return dict(rows=cfg["rows"], d=cfg["d"], experts=cfg["experts"], topk=cfg["topk"],
                inter=cfg["inter"], shared=cfg["shared"])


def tensor_specs(cfg):
    """(name, shape, dtype, stream, std) of every generated input tensor."""
    T, d, E, I, S = cfg["rows"], cfg["d"], cfg["experts"], cfg["inter"], cfg["shared"]
    ps = E + (1 if S > 0 else 0)
    specs = [
        ("x", (T, d), "f16", STREAM_X, STD_X),
        ("w_router", (ps, d), "f32", STREAM_W_ROUTER, STD_W),
        ("w_gate_up", (E, 2 * I, d), "f16", STREAM_W_GATE_UP, STD_W),
        ("w_down", (E, d, I), "f16", STREAM_W_DOWN, STD_W),
    ]
    if S > 0:
        specs += [
            ("w_sh_gate_up", (2 * S, d), "f16", STREAM_W_SH_GATE_UP, STD_W),
            ("w_sh_down", (d, S), "f16", STREAM_W_SH_DOWN, STD_W),
        ]
    return specs


def algorithmic_work(cfg, touched=None):
    """Algorithmic FLOPs and minimum HBM bytes per stage (padding excluded).

    touched: experts that received at least one token (all when None).
    """
    T, d, E, K, I, S = (cfg["rows"], cfg["d"], cfg["experts"], cfg["topk"], cfg["inter"], cfg["shared"])
    ps = E + (1 if S > 0 else 0)
    Et = E if touched is None else touched
    w = {}
    w["router_flops"] = 2 * T * d * ps
    w["router_bytes"] = T * d * 2 + ps * d * 4 + T * ps * 4
    w["route_bytes"] = T * E * 4 + T * K * 8
    w["gemm_flops"] = 6 * T * K * d * I + (6 * T * d * S if S else 0)
    w["gate_up_flops"] = 4 * T * K * d * I + (4 * T * d * S if S else 0)
    w["down_flops"] = 2 * T * K * d * I + (2 * T * d * S if S else 0)
    w["gate_up_bytes"] = Et * 2 * I * d * 2 + T * d * 2 + T * K * I * 2 + (2 * S * d * 2 + T * S * 2 if S else 0)
    w["down_bytes"] = Et * d * I * 2 + T * K * I * 2 + T * K * d * 2 + (d * S * 2 + T * S * 2 + T * d * 2 if S else 0)
    w["combine_bytes"] = T * K * d * 2 + T * K * 8 + T * d * 2 + (T * d * 2 if S else 0)
    w["weight_bytes"] = Et * 3 * d * I * 2 + (3 * d * S * 2 if S else 0)
    return w
