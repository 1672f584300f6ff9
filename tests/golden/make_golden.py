"""Writes the golden fixtures of this directory: seeded config inputs, regenerated on the CPU from the
seed by bundles_amd.synth (never stored), run through the C oracle; outputs saved as .npz (plain
arrays, load with allow_pickle=False).  The reference ships no test vectors, so these are the
build's own anchors: test_golden.py pins the oracle to them, test_gpu_golden.py the kernels.

    python tests/golden/make_golden.py          # rewrites tests/golden/*.npz
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)


def _h(t):
    import torch
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _f(t):
    return t.contiguous().numpy()


def moe_cfg1(O):
    """Config 1: int8 W8A8 MoE, 8 tokens, 512 experts top-10, seed 0."""
    from bundles_amd import synth
    M, E, k = 8, 512, 10
    d = synth.moe_inputs(M, "cpu", seed=0)
    x, wr, gw = _h(d["x"]), _h(d["router_w"]), _h(d["gate_w"])
    r = O.route(x, wr, k)
    used = np.unique(r["ids"])
    w13 = np.zeros((E, 1024, 2048), np.int8)
    s13 = np.zeros((E, 1024), np.float32)
    w2 = np.zeros((E, 2048, 512), np.int8)
    s2 = np.zeros((E, 2048), np.float32)
    for e in used:  # only the routed experts are read; the rest stay zero
        w13[e], s13[e] = O.quant_rows_i8(O.bf16_to_f32(_h(d["w13"][e])))
        w2[e], s2[e] = O.quant_rows_i8(O.bf16_to_f32(_h(d["w2"][e])))
    sw13, ss13 = O.quant_rows_i8(O.bf16_to_f32(_h(d["sw13"])))
    sw2, ss2 = O.quant_rows_i8(O.bf16_to_f32(_h(d["sw2"])))
    res = O.moe(0, x, wr, w13, s13, w2, s2, sw13, ss13, sw2, ss2, gw, k, debug=True)
    return dict(ids=res["ids"], wts=res["wts"], out=res["out"], h=res["h"],
                acc13_rowsum=res["acc13"].astype(np.int64).sum(1), acc13_head=res["acc13"][:, :16].copy(),
                acc2_rowsum=res["acc2"].astype(np.int64).sum(1), acc2_head=res["acc2"][:, :16].copy(),
                x_bits_sum=np.int64(x.astype(np.int64).sum()), used=used.astype(np.int32))


def gdn_b2(O):
    """Config 3 shape at 2 sequences x (1 + 4) positions, seed 0."""
    from bundles_amd import synth
    B, T = 2, 5
    d = synth.gdn_inputs(B, T, "cpu", seed=0)
    out, snaps, cs = O.gdn_verify(B, T, _h(d["mixed"]), _h(d["z"]), _h(d["a"]), _h(d["b"]), _h(d["conv_state"]),
                                  _h(d["conv_w"]), _f(d["A_log"]), _f(d["dt_bias"]), _f(d["S0"]), _h(d["norm_w"]),
                                  1e-6)
    return dict(out=out, snap_sum=snaps.astype(np.float64).sum(axis=(3, 4)),
                snap_slice=snaps[:, :, [0, 17], :4, :].copy(), conv_state=cs)


def attn_t4(O):
    """Config 4 shape at 4 tokens, seed 0 (weights quantized to e4m3 128x128 blocks by the oracle)."""
    from bundles_amd import synth
    T = 4
    d = synth.attn_inputs(T, "cpu", seed=0)
    wqkv = np.concatenate([O.bf16_to_f32(_h(d[n])) for n in ("wqg", "wk", "wv")], axis=0)
    q, s = O.quant_blocks_e4m3(wqkv)
    qo, so = O.quant_blocks_e4m3(O.bf16_to_f32(_h(d["wo"])))
    r = O.attn_proj(_h(d["x"]), q[:8192], s[:64], q[8192:8704], s[64:68], q[8704:], s[68:72], _h(d["q_norm_w"]),
                    _h(d["k_norm_w"]), 1e-6, _f(d["cos_sin"]), _f(d["positions"]))
    gate = r["gate"].reshape(T, 4096)
    out = O.attn_oproj(_h(d["attn"]), gate, qo, so)
    return dict(q=r["q"], gate=r["gate"], k=r["k"], v=r["v"], k8=r["k8"], v8=r["v8"], oproj=out,
                wqkv_sum=np.int64(q.astype(np.int64).sum()), positions=_f(d["positions"]))


def lmhead_r8(O):
    """Config 5 form at 8 rows x 4096 vocab, seed 0 (final norm, per-row int8, argmax)."""
    from bundles_amd import synth
    d = synth.lmhead_inputs(8, 4096, "cpu", seed=0)
    wq, ws = O.quant_rows_i8(O.bf16_to_f32(_h(d["w"])))
    ids, logits = O.lmhead(_h(d["h"]), _h(d["norm_w"]), 1e-6, wq, ws, want_logits=True)
    return dict(ids=ids, logits=logits, wq_sum=np.int64(wq.astype(np.int64).sum()))


FIXTURES = {"moe_cfg1_int8_m8": moe_cfg1, "gdn_b2_t5": gdn_b2, "attn_t4": attn_t4, "lmhead_r8_v4096": lmhead_r8}


def main():
    from oracle import oracle as O
    O.lib()
    for name, fn in FIXTURES.items():
        arrs = fn(O)
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **arrs)
        print(name, {k: v.shape for k, v in arrs.items()}, flush=True)


if __name__ == "__main__":
    main()
