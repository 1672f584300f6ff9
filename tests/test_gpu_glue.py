"""GPU parity of the hybrid layer's glue (q36_fp8_linear with segmented outputs, q36_add_rmsnorm)
against the CPU oracle.

Bar: the add-norm is bit-exact (residual and normalised rows: one fixed reduction order on both
sides); the fp8 linear is within the bf16 bar (1e-2 relative per row; the fp8 MFMA does not round
its block sums exactly), and its segments receive exactly the columns of the unsegmented call."""
import numpy as np
import pytest
import torch

from helpers import assert_bf16_close, bits16, np_

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def glue():
    from bundles_amd import _lib
    _lib.lib()
    from bundles_amd.qwen36_layer import glue
    return glue


@pytest.mark.parametrize("T,delta", [(1, True), (7, True), (256, True), (5, False)])
def test_add_rmsnorm_bit_exact(glue, oracle_mod, dev, T, delta):
    print(f"add_rmsnorm T={T} delta={delta}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(T)
    d = (torch.randn((T, 2048), generator=g) * 2).to(torch.bfloat16) if delta else None
    r = (torch.randn((T, 2048), generator=g) * 5).to(torch.bfloat16)
    w = (torch.randn(2048, generator=g) * 0.2).to(torch.bfloat16)
    rd = r.to(dev)
    out = glue.add_rmsnorm(None if d is None else d.to(dev), rd, w.to(dev), 1e-6)
    torch.cuda.synchronize()
    ro, rr = oracle_mod.add_rmsnorm(None if d is None else bits16(d), bits16(r), bits16(w), 1e-6)
    assert np.array_equal(bits16(rd), rr), "residual differs"
    assert np.array_equal(bits16(out), ro), "normalised rows differ"


@pytest.mark.parametrize("T,N,K", [(1, 2048, 4096), (37, 384, 2048), (256, 2048, 4096), (64, 12352, 2048)])
def test_fp8_linear_parity(glue, oracle_mod, dev, T, N, K):
    print(f"fp8_linear T={T} N={N} K={K}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(N + T)
    x = torch.randn((T, K), generator=g).to(torch.bfloat16).to(dev)
    w = glue.prepare_fp8_weight((torch.randn((N, K), generator=g) * 0.02).to(torch.bfloat16).to(dev))
    ws = glue.LinearWorkspace(T, K, dev)
    y = glue.fp8_linear(x, w, ws)
    torch.cuda.synchronize()
    ref = oracle_mod.fp8_linear(bits16(x), np_(w.q)[:], np_(w.s))[:, :N]
    wr, ar, er = assert_bf16_close(bits16(y), ref, 1e-2, "fp8_linear")
    print(f"row err {wr:.2e} elem {ar:.2e} exact {er:.4f}", flush=True)


@pytest.mark.parametrize("T,N,K", [(64, 9216, 2048), (150, 9216, 2048), (200, 12416, 2048), (256, 12416, 2048),
                                   (256, 2048, 4096)])
def test_fp8_linear_rows_do_not_depend_on_the_batch(glue, dev, T, N, K):
    """Rows 0..36 of a T-token call equal a 37-token call (the streaming GEMM) bit for bit.  Past 128
    tokens with K = 2048 the call takes the tiled GEMM (64-token groups at 150, 128-token groups at 200
    and 256, ragged last token tile at 150 and 200): both form fma(blocksum, xs * ws, acc) over the K
    blocks in order from zero, and each token is quantized on its own."""
    print(f"fp8_linear batch invariance T={T} N={N} K={K}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(T + K)
    x = torch.randn((T, K), generator=g).to(torch.bfloat16).to(dev)
    w = glue.prepare_fp8_weight((torch.randn((N, K), generator=g) * 0.02).to(torch.bfloat16).to(dev))
    big = glue.fp8_linear(x, w, glue.LinearWorkspace(T, K, dev))
    small = glue.fp8_linear(x[:37].contiguous(), w, glue.LinearWorkspace(37, K, dev))
    torch.cuda.synchronize()
    assert torch.equal(big[:37], small)
    assert torch.isfinite(big.float()).all()


@pytest.mark.parametrize("T", [24, 200])
def test_fp8_linear_segments_match_the_single_output(glue, dev, T):
    """The GDN in_proj split: q|k|v 8192, z 4096, b 32, a 32 (12352 columns, 12416 weight rows), the
    first segment written into a wider strided buffer; at 24 tokens through the streaming GEMM, at
    200 through the tiled one (ragged last token tile)."""
    print(f"fp8_linear segments T={T}", flush=True)
    K = 2048
    g = torch.Generator(device="cpu").manual_seed(3)
    x = torch.randn((T, K), generator=g).to(torch.bfloat16).to(dev)
    w = glue.prepare_fp8_weight((torch.randn((12352, K), generator=g) * 0.02).to(torch.bfloat16).to(dev))
    ws = glue.LinearWorkspace(T, K, dev)
    y = glue.fp8_linear(x, w, ws)
    wide = torch.full((T, 8192 + 64), 7.0, dtype=torch.bfloat16, device=dev)
    qkv = wide[:, :8192]
    z = torch.empty((T, 4096), dtype=torch.bfloat16, device=dev)
    b = torch.empty((T, 32), dtype=torch.bfloat16, device=dev)
    a = torch.empty((T, 32), dtype=torch.bfloat16, device=dev)
    glue.fp8_linear(x, w, ws, segments=[(0, qkv), (8192, z), (12288, b), (12320, a)])
    torch.cuda.synchronize()
    assert torch.equal(qkv, y[:, :8192]) and torch.equal(z, y[:, 8192:12288])
    assert torch.equal(b, y[:, 12288:12320]) and torch.equal(a, y[:, 12320:])
    assert torch.all(wide[:, 8192:] == 7.0), "a segment wrote past its columns"
    with pytest.raises(ValueError):
        glue.fp8_linear(x, w, ws, segments=[(0, qkv), (8192, z)])
