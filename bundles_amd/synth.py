"""Seeded synthetic inputs of the benchmark configurations (random-init weights, no checkpoints).

Every generator draws on the given device with its own torch.Generator so a run is
reproducible; the CPU checker receives copies of the same tensors.
Shapes follow the configurations: hidden 2048, 512 experts top-10 with intermediate 512 plus one
shared expert; GDN 16 QK heads x 128 and 32 V heads x 128; attention 16 q heads / 2 KV heads x 256;
vocab 151936.
"""
from __future__ import annotations

import math

import torch

H, E, TOPK, INTER = 2048, 512, 10, 512


def gen(device, seed: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def randn(shape, g, device, std=1.0, dtype=torch.bfloat16):
    return (torch.randn(shape, generator=g, device=device, dtype=torch.float32) * std).to(dtype)


def zipf_bias(E: int, s: float, g, device) -> torch.Tensor:
    """bias_e = ln p_e with p_e proportional to rank(e)^-s over a seeded permutation of the experts:
    adding it to the router logits multiplies the routing distribution by a Zipf(s) prior."""
    rank = torch.empty(E, dtype=torch.float32, device=device)
    perm = torch.randperm(E, generator=g, device=device)
    rank[perm] = torch.arange(1, E + 1, dtype=torch.float32, device=device)
    p = rank.pow(-s)
    return torch.log(p / p.sum())


def moe_inputs(M: int, device, seed: int = 0, E: int = E, H: int = H, I: int = INTER, zipf: float | None = None):
    """Config 1 / 2 MoE block: bf16 x ~ N(0,1), router N(0,0.02), experts and shared expert N(0,0.02)."""
    g = gen(device, seed)
    d = dict(
        x=randn((M, H), g, device),
        router_w=randn((E, H), g, device, 0.02),
        w13=randn((E, 2 * I, H), g, device, 0.02),
        w2=randn((E, H, I), g, device, 0.02),
        sw13=randn((2 * I, H), g, device, 0.02),
        sw2=randn((H, I), g, device, 0.02),
        gate_w=randn((H,), g, device, 0.02),
    )
    d["router_bias"] = zipf_bias(E, zipf, g, device) if zipf else None
    return d


def gdn_inputs(B: int = 32, T: int = 5, device="cpu", seed: int = 0):
    """Config 3 GDN verify step: mixed_qkv / z / a / b ~ N(0,1) drawn directly (bf16), conv state
    N(0,1), conv weights U(-1/2, 1/2) (fan-in 4), A_log = ln U[1,16], dt_bias = softplus^-1 of
    dt ~ logU[1e-3, 1e-1], state S0 ~ N(0, 0.1) fp32, norm weight N(1, 0.1)."""
    g = gen(device, seed)
    R = B * T
    dt = torch.exp(torch.rand(32, generator=g, device=device) * (math.log(1e-1) - math.log(1e-3)) + math.log(1e-3))
    return dict(
        B=B, T=T,
        mixed=randn((R, 8192), g, device),
        z=randn((R, 4096), g, device),
        a=randn((R, 32), g, device),
        b=randn((R, 32), g, device),
        conv_state=randn((B, 8192, 3), g, device),
        conv_w=((torch.rand((8192, 4), generator=g, device=device) - 0.5)).to(torch.bfloat16),
        A_log=torch.log(1 + 15 * torch.rand(32, generator=g, device=device)),
        dt_bias=dt + torch.log(-torch.expm1(-dt)),
        S0=torch.randn((B, 32, 128, 128), generator=g, device=device) * 0.1,
        norm_w=randn((128,), g, device, 0.1) + 1.0,
    )


def gdn_ring_inputs(B: int = 32, T: int = 4, device="cpu", seed: int = 0, wp=None, padded=()):
    """A ReplaySSM verify step: the config-3 front of gdn_inputs (mixed, z, a, b, conv weights,
    gates, norm weight) over the served pools.  Pools have a few spare slots and every index is a
    distinct random slot: checkpoint h0 [slots, 32, 128, 128] ~ N(0, 0.1), conv state N(0, 1),
    rings holding write_pos committed entries per request (wp: an int, or None for U[0, 16 - T])
    at a random cache_base: d ~ N(0, 0.3) bf16 with its low part, unit keys with their low part,
    g from the gate formula on a ~ N(0, 1).  Requests listed in `padded` get state_idx -1."""
    f = gdn_inputs(B, T, device, seed)
    g = gen(device, seed + 7919)
    slots, rslots, wslots = B + 3, B + 2, B + 1

    def pick(n):
        return torch.randperm(n, generator=g, device=device)[:B].to(torch.int64)

    state_idx, replay_idx, win_idx = pick(slots), pick(rslots), pick(wslots)
    for r in padded:
        state_idx[r] = -1
    if wp is None:
        write_pos = torch.randint(0, 16 - T + 1, (rslots,), generator=g, device=device, dtype=torch.int32)
    else:
        write_pos = torch.full((rslots,), int(wp), dtype=torch.int32, device=device)
    cache_base = torch.randint(0, 16, (rslots,), generator=g, device=device, dtype=torch.int32)
    d32 = torch.randn((rslots, 32, 16, 128), generator=g, device=device) * 0.3
    k32 = torch.randn((rslots, 16, 16, 128), generator=g, device=device)
    k32 = k32 / k32.norm(dim=-1, keepdim=True)
    d_ring = d32.to(torch.bfloat16)
    k_ring = k32.to(torch.bfloat16)
    xg = torch.randn((rslots, 32, 16), generator=g, device=device) + f["dt_bias"][None, :, None]
    g_ring = -torch.exp(f["A_log"])[None, :, None] * torch.nn.functional.softplus(xg)
    f.update(
        rows=B * T, slots=slots, rslots=rslots, wslots=wslots,
        conv_state=randn((slots, 8192, 3), g, device),
        window=torch.zeros((wslots, 8192, T + 2), dtype=torch.bfloat16, device=device),
        h0=torch.randn((slots, 32, 128, 128), generator=g, device=device) * 0.1,
        d_ring=d_ring, dlo_ring=(d32 - d_ring.float()).to(torch.bfloat16),
        k_ring=k_ring, klo_ring=(k32 - k_ring.float()).to(torch.bfloat16),
        g_ring=g_ring.contiguous(),
        qsl=torch.arange(0, (B + 1) * T, T, dtype=torch.int32, device=device),
        state_idx=state_idx, replay_idx=replay_idx, win_idx=win_idx,
        write_pos=write_pos, cache_base=cache_base,
        scale=128 ** -0.5,
    )
    del f["S0"]
    return f


def rope_cos_sin(max_pos: int, rot_dim: int = 64, theta: float = 1e7, device="cpu") -> torch.Tensor:
    """fp32 [max_pos, rot_dim]: cos | sin of pos * theta^(-2i/rot_dim), i < rot_dim/2, from fp64."""
    inv = theta ** (-torch.arange(0, rot_dim, 2, dtype=torch.float64) / rot_dim)
    ang = torch.arange(max_pos, dtype=torch.float64)[:, None] * inv[None, :]
    return torch.cat([ang.cos(), ang.sin()], dim=1).to(torch.float32).to(device)


def attn_inputs(T: int = 128, device="cpu", seed: int = 0, max_pos: int = 32768):
    """Config 4: x ~ N(0,1) [T,2048]; Wqg [8192,2048] (q|gate interleaved per head), Wk/Wv [512,2048],
    Wo [2048,4096] ~ N(0,0.02) bf16 (quantized to e4m3 blocks by the caller); q/k norm weights
    N(0,0.1) (Gemma (1+w) form); positions U[0, 32768); attention output N(0,1) [T,4096]."""
    g = gen(device, seed)
    return dict(
        x=randn((T, 2048), g, device),
        wqg=randn((8192, 2048), g, device, 0.02),
        wk=randn((512, 2048), g, device, 0.02),
        wv=randn((512, 2048), g, device, 0.02),
        wo=randn((2048, 4096), g, device, 0.02),
        q_norm_w=randn((256,), g, device, 0.1),
        k_norm_w=randn((256,), g, device, 0.1),
        positions=torch.randint(0, max_pos, (T,), generator=g, device=device, dtype=torch.int32),
        attn=randn((T, 4096), g, device),
        cos_sin=rope_cos_sin(max_pos, device=device),
    )


def lmhead_inputs(R: int = 2048, V: int = 151936, device="cpu", seed: int = 0):
    """Config 5 lm_head: hidden ~ N(0,1) [R,2048], final norm weight N(0,0.1), W ~ N(0,0.02) [V,2048]."""
    g = gen(device, seed)
    return dict(h=randn((R, 2048), g, device), norm_w=randn((2048,), g, device, 0.1),
                w=randn((V, 2048), g, device, 0.02))
