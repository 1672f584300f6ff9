"""GPU parity of the reference's prepare-time weight formats (libq36 through the C-ABI) against the
oracle, and the bridges into the nodes.

Bar: the q8-block-v1 and DENSE8 copies bit-exact (codes and fp16 scales); a q8-block-v1 copy imported
as the decode MoE's int8 experts gives a MoE block bit-exact with the oracle's on the copy's own codes
and scales (ids, output); an fp8 checkpoint's blocks consumed as they are give the fp8 MoE block
within the bf16 bar of the oracle's and the identical block when re-quantized on the GPU.
"""
import numpy as np
import pytest
import torch

from helpers import assert_bf16_close, bits16, np_

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def fmt():
    from bundles_amd import _lib
    _lib.lib()
    from bundles_amd.qwen36_layer import formats
    return formats


def _bf16_weights(shape, g, dev, std=0.02):
    return (torch.randn(shape, generator=g, device=dev) * std).to(torch.bfloat16)


@pytest.mark.parametrize("channel", [True, False])
def test_q8_block_v1_bit_exact(fmt, oracle_mod, dev, channel):
    print(f"q8-block-v1 channel={channel}", flush=True)
    g = torch.Generator(device=dev).manual_seed(3)
    E, H, I = 4, 2048, 512
    w13 = _bf16_weights((E, 2 * I, H), g, dev)
    w2 = _bf16_weights((E, H, I), g, dev)
    w13[1, 7] = 0                                      # a zero row: zero codes, zero scale
    w2[2, 5, :128] = torch.arange(128, device=dev).to(torch.bfloat16) * 0.5  # exact .5 ties
    blocks = fmt.quant_q8_block_v1(w13, w2, channel=channel)
    torch.cuda.synchronize()
    ref = oracle_mod.quant_q8_block_v1(w13.float().cpu().numpy(), w2.float().cpu().numpy(), channel=channel)
    assert np.array_equal(np_(blocks), ref)


def test_dense8_bit_exact_into_a_wider_scale_buffer(fmt, oracle_mod, dev):
    g = torch.Generator(device=dev).manual_seed(4)
    N, K = 384, 4096
    w = _bf16_weights((N, K), g, dev)
    w[10] = 0
    wide = torch.zeros((K // 128, N + 64), dtype=torch.float16, device=dev)
    q, s = fmt.quant_dense8(w, s=wide[:, 32:32 + N])
    torch.cuda.synchronize()
    rq, rs = oracle_mod.quant_dense8(w.float().cpu().numpy())
    assert np.array_equal(np_(q), rq)
    assert np.array_equal(np_(wide[:, 32:32 + N]).view(np.uint16), rs)
    assert not torch.any(wide[:, :32]) and not torch.any(wide[:, 32 + N:]), "columns outside the block untouched"


def test_moe_on_an_imported_q8_block_v1_copy(fmt, oracle_mod, dev):
    """The reference's channel-mode expert copy drives the int8 decode MoE as it is."""
    from bundles_amd import synth
    from bundles_amd.qwen36_layer import moe
    O = oracle_mod
    M, E, H, I = 16, 64, 2048, 512
    d = synth.moe_inputs(M, dev, seed=6, E=E, zipf=1.1)
    blocks = fmt.quant_q8_block_v1(d["w13"], d["w2"], channel=True)
    ew = moe.prepare_experts_q8_block_v1(blocks, H, I, d["sw13"], d["sw2"])
    ws = moe.Workspace(E, H, I, 10, moe.Q36_MOE_INT8, dev)
    out = moe.moe_row_batch(d["x"], None, d["router_w"], d["gate_w"], ew, 10, ws, router_bias=d["router_bias"])
    torch.cuda.synchronize()
    # the oracle on the copy's own codes and scales (fp16 scales widened exactly)
    hb = np_(blocks)
    q13 = np.stack([O.q8_block_parts(hb[e], H, I)[0] for e in range(E)])
    q2 = np.stack([O.q8_block_parts(hb[e], H, I)[1] for e in range(E)])
    c13 = np.stack([O.q8_block_parts(hb[e], H, I)[2][:, 0] for e in range(E)])
    c2 = np.stack([O.q8_block_parts(hb[e], H, I)[3][:, 0] for e in range(E)])
    f16 = lambda b: torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.float16).float().numpy()
    assert np.array_equal(moe.unpack_frag8_np(np_(ew.w13)), q13) and np.array_equal(moe.unpack_frag8_np(np_(ew.w2)), q2)
    assert np.array_equal(np_(ew.s13), f16(c13)) and np.array_equal(np_(ew.s2), f16(c2))
    r = O.moe(0, bits16(d["x"]), bits16(d["router_w"]), q13, f16(c13), q2, f16(c2),
              moe.unpack_frag8_np(np_(ew.sw13)), np_(ew.ss13), moe.unpack_frag8_np(np_(ew.sw2)), np_(ew.ss2),
              bits16(d["gate_w"]), 10, bias=np_(d["router_bias"]))
    assert np.array_equal(np_(ws.views(M)["ids"]), r["ids"])
    assert np.array_equal(bits16(out), r["out"]), "int8 MoE on the imported copy: bit-exact"


def test_moe_on_fp8_checkpoint_blocks(dev, oracle_mod):
    """Pre-quantized e4m3 128x128 blocks (an fp8 checkpoint's weight / weight_scale_inv, here made by the
    CPU oracle) consumed as they are: the same block as re-quantizing the bf16 weights on the GPU."""
    from bundles_amd import synth
    from bundles_amd.qwen36_layer import moe
    O = oracle_mod
    M, E = 16, 64
    d = synth.moe_inputs(M, dev, seed=8, E=E, zipf=1.1)

    def ckpt(w):
        q, s = [], []
        for m in w.float().cpu().numpy().reshape(-1, *w.shape[-2:]):
            qq = np.zeros(m.shape, np.uint8)
            ss = np.zeros((m.shape[0] // 128, m.shape[1] // 128), np.float32)
            O.lib().q36o_quant_blocks_e4m3(O._p(np.ascontiguousarray(m)), m.shape[0], m.shape[1], O._p(qq), O._p(ss))
            q.append(qq)
            s.append(ss)
        q = torch.from_numpy(np.stack(q).reshape(w.shape)).to(dev)
        s = torch.from_numpy(np.stack(s).reshape(*w.shape[:-2], w.shape[-2] // 128, w.shape[-1] // 128)).to(dev)
        return q.view(torch.float8_e4m3fn), s

    parts = [ckpt(d[k]) for k in ("w13", "w2", "sw13", "sw2")]
    ew = moe.prepare_experts_fp8_blocks(*(t for p in parts for t in p))
    ew_gpu = moe.prepare_experts(d["w13"], d["w2"], d["sw13"], d["sw2"], moe.Q36_MOE_FP8)
    ws = moe.Workspace(E, 2048, 512, 10, moe.Q36_MOE_FP8, dev)
    out = moe.moe_row_batch(d["x"], None, d["router_w"], d["gate_w"], ew, 10, ws, router_bias=d["router_bias"]).clone()
    out2 = moe.moe_row_batch(d["x"], None, d["router_w"], d["gate_w"], ew_gpu, 10, ws, router_bias=d["router_bias"])
    torch.cuda.synchronize()
    assert torch.equal(out, out2), "checkpoint blocks and GPU-quantized blocks give the same block"
    r = O.moe(1, bits16(d["x"]), bits16(d["router_w"]), *(np_(t.view(torch.uint8)) if i % 2 == 0 else np_(t)
                                                          for p in parts for i, t in enumerate(p)),
              bits16(d["gate_w"]), 10, bias=np_(d["router_bias"]))
    assert_bf16_close(bits16(out), r["out"], 1e-2, "fp8 MoE on checkpoint blocks")
