"""Benchmark configurations and seeded synthetic inputs.

The generator is the counter-based SplitMix64 stream declared in
include/raggedroute_capi.h (rr_fill_uniform / rr_fill_normal): element i of
sub-stream s under seed `seed` is z = splitmix64(seed*G + s*H + i) with
G = 0x9E3779B97F4A7C15, H = 0xD1B54A32D192ED03 and
splitmix64(x) = mix(x + G). Uniform: low + (high - low) * (z >> 40) * 2^-24
(float32, separately rounded). Normal: Box-Muller in float64 on
u1 = ((z >> 40) + 1) * 2^-24, u2 = ((z >> 16) & 0xFFFFFF) * 2^-24, rounded to
float32. The HIP fills and these numpy versions produce the same streams, so
multi-GB inputs are generated in HBM while small cases stay checkable on the
host. Routing ids use float64 uniforms u = (z >> 11) * 2^-53.

The configurations are the ones the benchmark and the parity tests use (role
of the reference's suites, reference configs/project/benchmark/*.json, at the
shapes of this build's measurement plan).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
STREAM_MUL = np.uint64(0xD1B54A32D192ED03)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)

# sub-stream ids of the tensors of one workload
S_X, S_ROUTER, S_EXPERTS, S_LOGITS, S_IDS, S_WEIGHTS, S_PERM, S_TIES, S_YPERM = range(1, 10)


def splitmix64(x: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = x.astype(np.uint64) + GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def stream_bits(count: int, seed: int, stream: int, start: int = 0) -> np.ndarray:
    with np.errstate(over="ignore"):
        base = np.uint64(seed) * GOLDEN + np.uint64(stream) * STREAM_MUL
        idx = np.arange(start, start + count, dtype=np.uint64)
        return splitmix64(base + idx)


def uniform(count: int, seed: int, stream: int, low: float = -1.0, high: float = 1.0) -> np.ndarray:
    z = stream_bits(count, seed, stream)
    u = (z >> np.uint64(40)).astype(np.float32) * np.float32(2.0**-24)
    return (np.float32(low) + np.float32(high - low) * u).astype(np.float32)


def normal(count: int, seed: int, stream: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    z = stream_bits(count, seed, stream)
    u1 = ((z >> np.uint64(40)) + np.uint64(1)).astype(np.float64) * 2.0**-24
    u2 = ((z >> np.uint64(16)) & np.uint64(0xFFFFFF)).astype(np.float64) * 2.0**-24
    n = np.sqrt(-2.0 * np.log(u1)) * np.cos(6.283185307179586 * u2)
    return (np.float64(np.float32(mean)) + np.float64(np.float32(std)) * n).astype(np.float32)


def unit_doubles(count: int, seed: int, stream: int, start: int = 0) -> np.ndarray:
    z = stream_bits(count, seed, stream, start)
    return (z >> np.uint64(11)).astype(np.float64) * 2.0**-53


def seeded_permutation(n: int, seed: int, stream: int) -> np.ndarray:
    return np.argsort(unit_doubles(n, seed, stream), kind="stable").astype(np.int64)


def zipf_draw(u: np.ndarray, n: int, s: float) -> np.ndarray:
    """Inverse-CDF draw of p(e) ~ (e + 1)^-s over e in [0, n)."""
    p = np.arange(1, n + 1, dtype=np.float64) ** (-s)
    cdf = np.cumsum(p / p.sum())
    cdf[-1] = 1.0
    return np.minimum(np.searchsorted(cdf, u, side="right"), n - 1).astype(np.int32)


def distinct_pairs(tokens: int, n: int, s: float | None, seed: int, stream: int) -> np.ndarray:
    """Per-token two distinct experts in [0, n): uniform (s None) or Zipf(s);
    the second draw is redrawn from fresh counters until it differs."""
    def draw(u):
        return (np.minimum((u * n).astype(np.int64), n - 1).astype(np.int32) if s is None
                else zipf_draw(u, n, s))
    first = draw(unit_doubles(tokens, seed, stream, 0))
    second = draw(unit_doubles(tokens, seed, stream, tokens))
    start = 2 * tokens
    bad = np.nonzero(second == first)[0]
    while bad.size:
        second[bad] = draw(unit_doubles(bad.size, seed, stream, start))
        start += bad.size
        bad = bad[second[bad] == first[bad]]
    return np.stack([first, second], axis=1)


@dataclass(frozen=True)
class ChainConfig:
    name: str
    tokens: int
    experts: int
    hidden: int
    output: int
    from_tokens: bool = True
    logit_bias_s: float | None = None  # log-Zipf expert bias strength (None: no bias)
    tie_fraction: float = 0.0          # chain_from_logits: rows with exact top-2/top-3 ties

    @property
    def routes(self) -> int:
        return 2 * self.tokens


# Measurement-plan configurations (C1..C5 and the headline).
C1 = ChainConfig("C1", 512, 32, 256, 64)
HEADLINE = ChainConfig("headline", 4096, 64, 256, 128)
C2 = ChainConfig("C2", 4096, 64, 256, 128, from_tokens=False, logit_bias_s=1.1, tie_fraction=0.02)
C5 = ChainConfig("C5", 16384, 128, 2048, 768, logit_bias_s=1.0)
CHAIN_CONFIGS = {c.name: c for c in (C1, HEADLINE, C2, C5)}


def expert_bias(experts: int, s: float, seed: int) -> np.ndarray:
    """bias[e] = -s * ln(pi(e) + 1) for a seeded expert permutation pi (log-Zipf(s))."""
    rank = seeded_permutation(experts, seed, S_PERM)
    return (-s * np.log(rank.astype(np.float64) + 1.0)).astype(np.float32)


def chain_inputs(cfg: ChainConfig, seed: int = 0) -> dict:
    """Host (numpy) inputs of a chain workload.

    chain_from_tokens: X ~ N(0,1), router W ~ N(0, 1/K), expert W ~ N(0, 1/K).
    With a logit bias, X[:, K-1] = 1 and router W[K-1, :] = bias, so
    X @ W_r carries the bias inside the same GEMM.
    chain_from_logits: logits ~ N(0,1) + bias[e]; in a seeded tie_fraction of
    the rows the 3rd-largest logit is set bit-equal to the 2nd.
    """
    t, e, k, n = cfg.tokens, cfg.experts, cfg.hidden, cfg.output
    sd = 1.0 / np.sqrt(k)
    x = normal(t * k, seed, S_X).reshape(t, k)
    we = normal(e * k * n, seed, S_EXPERTS, 0.0, sd).reshape(e, k, n)
    out = {"x": x, "expert_weights": we}
    if cfg.from_tokens:
        wr = normal(k * e, seed, S_ROUTER, 0.0, sd).reshape(k, e)
        if cfg.logit_bias_s is not None:
            x[:, k - 1] = 1.0
            wr[k - 1, :] = expert_bias(e, cfg.logit_bias_s, seed)
        out["router_weights"] = wr
    else:
        logits = normal(t * e, seed, S_LOGITS).reshape(t, e)
        if cfg.logit_bias_s is not None:
            logits = (logits + expert_bias(e, cfg.logit_bias_s, seed)[None, :]).astype(np.float32)
        if cfg.tie_fraction > 0:
            rows = np.nonzero(unit_doubles(t, seed, S_TIES) < cfg.tie_fraction)[0]
            order = np.argsort(-logits[rows], axis=1, kind="stable")
            logits[rows, order[:, 2]] = logits[rows, order[:, 1]]
            out["tie_rows"] = rows
        out["logits"] = logits
    return out


def route_ids(routes: int, experts: int, distribution: str, seed: int, s: float = 1.5) -> np.ndarray:
    """Histogram stress ids (C3): 'uniform', or 'hot50' = one seeded hot expert
    with p = 0.5 and Zipf(s) over the remaining experts. E = 1 gives all zeros."""
    if experts == 1:
        return np.zeros(routes, np.int32)
    u = unit_doubles(routes, seed, S_IDS)
    if distribution == "uniform":
        return np.minimum((u * experts).astype(np.int64), experts - 1).astype(np.int32)
    if distribution != "hot50":
        raise ValueError(distribution)
    hot = int(seeded_permutation(experts, seed, S_PERM)[0])
    others = np.array([x for x in range(experts) if x != hot], np.int32)
    v = unit_doubles(routes, seed, S_IDS, routes)
    rest = others[zipf_draw(v, experts - 1, s)]
    return np.where(u < 0.5, hot, rest).astype(np.int32)


def c4_routing(tokens: int, experts: int, active: int, s: float, seed: int):
    """Per-token two distinct experts ~ Zipf(s) over the first `active` experts
    (the rest stay empty) and weights = softmax of two N(0,1) draws."""
    ids = distinct_pairs(tokens, active, s, seed, S_IDS)
    g = normal(2 * tokens, seed, S_WEIGHTS).reshape(tokens, 2).astype(np.float64)
    g = np.exp(g - g.max(axis=1, keepdims=True))
    w = (g / g.sum(axis=1, keepdims=True)).astype(np.float32)
    assert experts >= active
    return ids.astype(np.int32), w


def chain_inputs_device(cfg: ChainConfig, seed: int, device) -> dict:
    """Same tensors as chain_inputs, generated in HBM by rr_fill_normal
    (torch tensors; torch is only the allocator here). chain_from_tokens only."""
    import torch
    import raggedroute_amd as rr

    if not cfg.from_tokens:
        raise ValueError("device generation covers chain_from_tokens inputs")
    t, e, k, n = cfg.tokens, cfg.experts, cfg.hidden, cfg.output
    sd = float(np.float32(1.0 / np.sqrt(k)))
    stream = torch.cuda.current_stream(device).cuda_stream
    x = torch.empty(t, k, device=device)
    we = torch.empty(e, k, n, device=device)
    wr = torch.empty(k, e, device=device)
    for tensor, sid, std in ((x, S_X, 1.0), (we, S_EXPERTS, sd), (wr, S_ROUTER, sd)):
        if rr.fill_normal(tensor.data_ptr(), tensor.numel(), seed, sid, 0.0, std, stream) != 0:
            raise RuntimeError("rr_fill_normal failed")
    if cfg.logit_bias_s is not None:
        x[:, k - 1] = 1.0
        wr[k - 1, :] = torch.from_numpy(expert_bias(e, cfg.logit_bias_s, seed)).to(device)
    return {"x": x, "expert_weights": we, "router_weights": wr}


# ---- post-route chain (chain_from_route_ids) ----

ROUTE_DISTRIBUTIONS = ("uniform", "zipf", "single_hot", "round_robin", "duplicate_route")


def topk_route_ids(tokens: int, top_k: int, experts: int, distribution: str, seed: int,
                   s: float = 1.4) -> np.ndarray:
    """[tokens, top_k] expert ids with the distributions of reference
    include/raggedroute/benchmark/adapter_utils.h:206-248: uniform / zipf
    (p ~ (e + 1)^-s) draws redrawn until distinct inside the token;
    single_hot = rank; round_robin = (token + rank) mod E; duplicate_route =
    all zeros. Draws come from this module's counter stream, not mt19937_64."""
    if tokens < 1 or top_k < 1 or experts < top_k:
        raise ValueError("route shape requires tokens>=1 and experts>=top_k>=1")
    rank = np.arange(top_k, dtype=np.int64)[None, :]
    token = np.arange(tokens, dtype=np.int64)[:, None]
    if distribution == "duplicate_route":
        return np.zeros((tokens, top_k), np.int32)
    if distribution == "single_hot":
        return np.broadcast_to(rank, (tokens, top_k)).astype(np.int32)
    if distribution == "round_robin":
        return ((token + rank) % experts).astype(np.int32)
    if distribution not in ("uniform", "zipf"):
        raise ValueError(f"unsupported distribution: {distribution}")

    def draw(u):
        return (np.minimum((u * experts).astype(np.int64), experts - 1).astype(np.int32)
                if distribution == "uniform" else zipf_draw(u, experts, s))

    ids = np.empty((tokens, top_k), np.int32)
    start = 0
    for r in range(top_k):
        col = draw(unit_doubles(tokens, seed, S_IDS, start))
        start += tokens
        bad = np.nonzero((ids[:, :r] == col[:, None]).any(axis=1))[0]
        while bad.size:
            col[bad] = draw(unit_doubles(bad.size, seed, S_IDS, start))
            start += bad.size
            bad = bad[(ids[bad, :r] == col[bad, None]).any(axis=1)]
        ids[:, r] = col
    return ids


def topk_route_weights(tokens: int, top_k: int, seed: int) -> np.ndarray:
    """U(0.01, 1) weights normalised per token in float32, rank order
    (reference benchmarks/adapters/postroute_chain_adapter.cpp:684-694)."""
    w = uniform(tokens * top_k, seed, S_WEIGHTS, 0.01, 1.0).reshape(tokens, top_k)
    out = np.empty_like(w)
    total = np.zeros(tokens, np.float32)
    for r in range(top_k):
        total = (total + w[:, r]).astype(np.float32)
    for r in range(top_k):
        out[:, r] = (w[:, r] / total).astype(np.float32)
    return out


@dataclass(frozen=True)
class RouteChainConfig:
    name: str
    tokens: int
    experts: int
    hidden: int
    output: int
    top_k: int
    distribution: str = "uniform"
    zipf_s: float = 1.4

    @property
    def routes(self) -> int:
        return self.tokens * self.top_k


def route_chain_configs() -> dict:
    """The reference's post-route release cases
    (configs/project/benchmark/six_ops_v4_postroute_release.json): small
    T64/E16/K64/N64, representative T512/E64/K128/N128, large
    T2048/E64/K128/N128 for top_k 2, 4, 8, and max_route_pairs
    T8192/E64/K64/N64 top_k 8."""
    out = {}
    for name, t, e, k, n in (("small", 64, 16, 64, 64), ("representative", 512, 64, 128, 128),
                             ("large", 2048, 64, 128, 128)):
        for top_k in (2, 4, 8):
            cfg = RouteChainConfig(f"{name}.topk{top_k}", t, e, k, n, top_k)
            out[cfg.name] = cfg
    out["max_route_pairs.topk8"] = RouteChainConfig("max_route_pairs.topk8", 8192, 64, 64, 64, 8)
    return out


def route_chain_inputs(cfg: RouteChainConfig, seed: int = 0) -> dict:
    """Host inputs: X ~ U(-1, 1), expert W ~ U(-1, 1) (the reference's
    make_random_floats range), ids and weights as above."""
    t, e, k, n = cfg.tokens, cfg.experts, cfg.hidden, cfg.output
    return {
        "x": uniform(t * k, seed, S_X).reshape(t, k),
        "expert_weights": uniform(e * k * n, seed, S_EXPERTS).reshape(e, k, n),
        "ids": topk_route_ids(t, cfg.top_k, e, cfg.distribution, seed, cfg.zipf_s),
        "weights": topk_route_weights(t, cfg.top_k, seed),
    }
