"""Seeded synthetic Q/K/V for the prefill benchmark configurations.

The reference measures on Q/K captured from Llama-3.1-8B after RoPE
(eval/efficiency/capture_qk_real.py:69-114) and random V
(eval/efficiency/benchmark_attention_multilayer.py:143-144).  No weights are
available offline, so inputs are generated with a fixed recipe:

  1. One CPU ``torch.Generator`` seeded with ``seed`` draws, in this order,
     Q [1,Hq,L,D], K [1,Hkv,L,D] and V [1,Hkv,L,D] ~ N(0,1) in fp32.
  2. RoPE, rotate-half convention (capture_qk_real.py:45-56), is applied to Q
     and K with inv_freq = 1 / theta^(2i/D) and angle = position * inv_freq.
  3. Structure is added to K after RoPE:
       - sinks: the first ``n_sinks`` tokens are scaled by ``sink_scale``;
       - vertical stripes: ``round(stripe_density * L)`` positions drawn by
         ``randperm`` get a shared per-KV-head direction of norm
         ``stripe_norm`` added;
       - slash diagonals: ``periodic_amp * (cos(2 pi t / P) e_a + sin(2 pi t / P) e_b)``
         with e_a, e_b an orthonormal pair per KV head.
     The stripe direction and the (e_a, e_b) pair are drawn after V from the
     same generator.
  4. All three tensors are cast to ``dtype``.

Generation runs on the CPU generator so the numbers do not depend on the GPU.
"""
from __future__ import annotations

import hashlib
import math
from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class SynthConfig:
    name: str
    L: int
    Hq: int
    Hkv: int
    D: int = 128
    dtype: torch.dtype = torch.bfloat16
    theta: float = 500000.0
    stripe_density: float = 0.01
    period: int = 256
    block_size: int = 128


# BASELINE.json configs (C4 reuses the C2 layer shape inside a full model).
CONFIGS = {
    "c0": SynthConfig("c0", 8192, 4, 1, dtype=torch.float32),
    "c1": SynthConfig("c1", 32768, 32, 8),
    "c2": SynthConfig("c2", 131072, 32, 8, stripe_density=0.005, period=512),
    "c3a": SynthConfig("c3a", 65536, 28, 4, theta=1000000.0, block_size=64),
    "c3b": SynthConfig("c3b", 65536, 28, 4, theta=1000000.0, block_size=128),
}


def _rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def make_qkv(L: int, Hq: int, Hkv: int, D: int = 128, dtype=torch.bfloat16, seed: int = 0,
             theta: float = 500000.0, stripe_density: float = 0.01, period: int = 256,
             n_sinks: int = 4, sink_scale: float = 6.0, stripe_norm: float = 3.0,
             periodic_amp: float = 2.0, chunk: int = 16384):
    """Returns (q [1,Hq,L,D], k [1,Hkv,L,D], v [1,Hkv,L,D]) on the CPU."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    q = torch.randn(1, Hq, L, D, generator=g)
    k = torch.randn(1, Hkv, L, D, generator=g)
    v = torch.randn(1, Hkv, L, D, generator=g)
    n_str = max(1, int(round(stripe_density * L)))
    pos = torch.randperm(L, generator=g)[:n_str]
    u = torch.randn(Hkv, D, generator=g)
    u = u / u.norm(dim=-1, keepdim=True) * stripe_norm
    ea = torch.randn(Hkv, D, generator=g)
    eb = torch.randn(Hkv, D, generator=g)
    ea = ea / ea.norm(dim=-1, keepdim=True)
    eb = eb - (eb * ea).sum(-1, keepdim=True) * ea
    eb = eb / eb.norm(dim=-1, keepdim=True)
    # RoPE in chunks of positions to bound temporaries at long L
    for t0 in range(0, L, chunk):
        t1 = min(L, t0 + chunk)
        cos, sin = _cos_sin_range(t0, t1, D, theta)
        for x in (q, k):
            xs = x[:, :, t0:t1]
            xs.copy_(xs * cos + _rotate_half(xs) * sin)
    k[:, :, :n_sinks] *= sink_scale
    k[0, :, pos, :] += u[:, None, :]
    t = torch.arange(L, dtype=torch.float64)
    ang = 2.0 * math.pi * t / period
    ca = torch.cos(ang).float()
    sa = torch.sin(ang).float()
    for t0 in range(0, L, chunk):
        t1 = min(L, t0 + chunk)
        k[0, :, t0:t1, :] += periodic_amp * (ca[None, t0:t1, None] * ea[:, None, :]
                                             + sa[None, t0:t1, None] * eb[:, None, :])
    return q.to(dtype), k.to(dtype), v.to(dtype)


def _cos_sin_range(t0: int, t1: int, D: int, theta: float):
    inv_freq = 1.0 / (theta ** (torch.arange(0, D, 2, dtype=torch.int64).float() / D))
    ang = torch.arange(t0, t1, dtype=torch.float32)[:, None] * inv_freq[None, :]
    emb = torch.cat([ang, ang], dim=-1)
    return emb.cos(), emb.sin()


def make_config(cfg: SynthConfig | str, seed: int = 0, L: int | None = None):
    """Inputs for a named BASELINE config (optionally at a shorter length)."""
    if isinstance(cfg, str):
        cfg = CONFIGS[cfg]
    return make_qkv(L or cfg.L, cfg.Hq, cfg.Hkv, cfg.D, cfg.dtype, seed, cfg.theta,
                    cfg.stripe_density, cfg.period)


def sha256_of(*tensors) -> str:
    h = hashlib.sha256()
    for t in tensors:
        t = t.contiguous()
        h.update(str(t.dtype).encode())
        h.update(str(tuple(t.shape)).encode())
        h.update(t.view(torch.uint8).numpy().tobytes())
    return h.hexdigest()


def c4_model_config(num_hidden_layers: int = 32, max_position_embeddings: int = 131072):
    """BASELINE config 4's model: a Llama-3.1-8B-shaped transformers
    LlamaConfig (hidden 4096, 32 query / 8 KV heads, head_dim 128, MLP 14336,
    vocabulary 128256, llama3 RoPE scaling with theta 500000), for random-init
    weights (no checkpoint is available offline)."""
    from transformers import LlamaConfig
    return LlamaConfig(hidden_size=4096, intermediate_size=14336, num_hidden_layers=num_hidden_layers,
                       num_attention_heads=32, num_key_value_heads=8, head_dim=128, vocab_size=128256,
                       max_position_embeddings=max_position_embeddings, rms_norm_eps=1e-5, tie_word_embeddings=False,
                       rope_parameters={"rope_type": "llama3", "rope_theta": 500000.0, "factor": 8.0,
                                        "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                                        "original_max_position_embeddings": 8192})
