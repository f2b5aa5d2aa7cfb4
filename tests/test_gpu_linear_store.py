"""GPU parity: device self-check, indexer-K store, fp8 dequant and GEMV.

Bit-exact for the store and the dequant (oracle: oracle/dsa_oracle.py);
GEMV within fp16 output rounding of the fp64 oracle (small shapes) or of an
fp32 matmul over exactly decoded weights (full BASELINE shapes).
"""
import pytest
import torch

from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu


def test_selfcheck(pkg, lib, dev):
    torch.cuda.synchronize()
    rc = lib.mi355_dsa_selfcheck(None)
    msg = pkg._lib.last_error()
    print(msg, flush=True)
    assert rc == 0, msg


@pytest.mark.parametrize("n_tok,page,nblk", [(1, 64, 2), (333, 64, 8), (4096, 16, 300),
                                             (65536, 64, 1100)])  # C5b: 64k tokens
def test_k_store_fp16(ops, dev, n_tok, page, nblk):
    g = torch.Generator().manual_seed(n_tok)
    k = torch.randn(n_tok, 128, generator=g).to(torch.float16)
    slot = torch.randperm(page * nblk, generator=g)[:n_tok].to(torch.int32)
    slot[::7] = -1          # graph padding
    slot[3::11] = page * nblk + 5  # beyond the cache
    kc = torch.randn(nblk, page, 128, generator=g).to(torch.float16)
    kd = kc.to(dev)
    ops.sm70_indexer_k_store(kd, k.to(dev), slot.to(dev))
    assert torch.equal(kd.cpu(), O.indexer_k_store(kc, k, slot))


@pytest.mark.parametrize("n_tok", [1, 15, 16, 17, 1000, 65536])
def test_k_store_fp8(ops, dev, n_tok):
    g = torch.Generator().manual_seed(n_tok)
    page = 64
    nblk = (n_tok + page - 1) // page + 3
    k = torch.randn(n_tok, 128, generator=g)
    k[::5] *= 300.0   # large magnitudes
    k[1::9] *= 1e-4   # small magnitudes: denormal codes
    k[2::13] = 0.0    # amax 0 -> FLT_MIN scale
    k = k.to(torch.float16)
    slot = torch.randperm(page * nblk, generator=g)[:n_tok].to(torch.int32)
    slot[::17] = -1
    kc = torch.randint(0, 256, (nblk, page, 132), generator=g, dtype=torch.int32).to(torch.uint8)
    kd = kc.to(dev)
    ops.sm70_indexer_k_store(kd, k.to(dev), slot.to(dev))
    assert torch.equal(kd.cpu(), O.indexer_k_store(kc, k, slot))


def test_k_store_fp8_ties_and_saturation(ops, dev):
    # rows whose scaled values hit e4m3 rounding ties exactly
    k = torch.zeros(4, 128)
    k[:, 0] = 448.0                                    # scale = 1
    k[0, 1:9] = torch.tensor([1.0625, 1.1875, 2.0 ** -10, 3 * 2.0 ** -10, 7.5 * 2.0 ** -9,
                              -1.0625, 240.0, 0.1])
    k[1, 1] = -448.0
    k[1, 2] = -0.0                                     # keeps its sign: code 0x80
    k[2, 1:] = torch.linspace(-447, 447, 127)
    k[3, 0] = 65504.0                                  # fp16 max
    k = k.to(torch.float16)
    slot = torch.arange(4, dtype=torch.int32)
    kc = torch.zeros(1, 4, 132, dtype=torch.uint8)
    kd = kc.to(dev)
    ops.sm70_indexer_k_store(kd, k.to(dev), slot.to(dev))
    assert torch.equal(kd.cpu(), O.indexer_k_store(kc, k, slot))


@pytest.mark.parametrize("N,K", [(8, 16), (136, 272), (2112, 6144), (384, 1040)])
def test_dequant_bitexact(ops, dev, N, K):
    g = torch.Generator().manual_seed(N + K)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.float16)
    q8, s = O.attn_fp8_quantize(w)
    out = torch.empty(N, K, dtype=torch.float16, device=dev)
    ops.sm70_attn_fp8_dequant(out, q8.to(dev), s.to(dev))
    assert torch.equal(out.cpu(), O.attn_fp8_dequant(q8, s))


def test_dequant_all_codes_extreme_scales(ops, dev):
    codes = torch.tensor([b for b in range(256) if (b & 0x7F) != 0x7F] * 2, dtype=torch.int32)
    w = codes[:256].to(torch.uint8).view(1, 256).repeat(256, 1).contiguous()
    s = torch.tensor([[1e-7, 3.0], [65504.0 / 448, 2.0 ** -20]], dtype=torch.float32)
    out = torch.empty(256, 256, dtype=torch.float16, device=dev)
    ops.sm70_attn_fp8_dequant(out, w.to(dev), s.to(dev))
    assert torch.equal(out.cpu(), O.attn_fp8_dequant(w, s))


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8])
@pytest.mark.parametrize("N,K", [(8, 16), (264, 400), (2112, 6144), (4104, 1024)])
def test_gemv_small(ops, dev, M, N, K):
    g = torch.Generator().manual_seed(M * 1000 + N + K)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.float16)
    q8, s = O.attn_fp8_quantize(w)
    x = torch.randn(M, K, generator=g).to(torch.float16)
    y = torch.empty(M, N, dtype=torch.float16, device=dev)
    ops.sm70_attn_fp8_gemv(y, x.to(dev), q8.to(dev), s.to(dev))
    ref = O.attn_fp8_gemv(x, q8, s)
    err = (y.cpu().double() - ref).abs()
    # fp16 output rounding of an fp32-accumulated exact-product sum
    assert (err <= ref.abs() * 2.0 ** -10 + 1e-3 * ref.abs().max()).all(), err.max()


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5])
@pytest.mark.parametrize("N,K", [(1032, 8192), (8, 16384), (2056, 12288)])
def test_gemv_long_k(ops, dev, M, N, K):
    """Long-K shapes (the LDS-ring kernel for M <= 4): a row count that is a
    multiple of 8 but not of 16, a single 8-row workgroup, and more k blocks
    than the ring's waves x depth; M = 5 takes the register kernel."""
    g = torch.Generator().manual_seed(M * 7 + N + K)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.float16)
    q8, s = O.attn_fp8_quantize(w)
    x = torch.randn(M, K, generator=g).to(torch.float16)
    y = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
    ops.sm70_attn_fp8_gemv(y, x.to(dev), q8.to(dev), s.to(dev))
    ref = O.attn_fp8_gemv(x, q8, s)
    err = (y.cpu().double() - ref).abs()
    assert (err <= ref.abs() * 2.0 ** -10 + 1e-3 * ref.abs().max()).all(), err.max()


def _decode_table(dev):
    return O.e4m3_decode(torch.arange(256, dtype=torch.int32).to(torch.uint8)).to(dev)


@pytest.mark.parametrize("N,K", [(24576, 6144), (6144, 24576), (2112, 6144)])
def test_gemv_baseline_shapes(ops, dev, N, K):
    """Full config C5a shapes against an fp32 GPU matmul over exactly decoded
    weights (torch, not the kernel under test)."""
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    wq = torch.randint(0, 256, (N, K), generator=g, device=dev, dtype=torch.int32)
    wq = torch.where((wq & 0x7F) == 0x7F, wq - 1, wq).to(torch.uint8)  # no NaN codes
    s = torch.rand((N + 127) // 128, (K + 127) // 128, generator=g, device=dev) * 1e-4
    table = _decode_table(dev)
    w32 = table[wq.long()] * s.repeat_interleave(128, 0)[:N].repeat_interleave(128, 1)[:, :K]
    for M in (1, 2, 3, 4):
        x = torch.randn(M, K, generator=g, device=dev).to(torch.float16)
        y = torch.empty(M, N, dtype=torch.float16, device=dev)
        ops.sm70_attn_fp8_gemv(y, x, wq, s)
        ref = x.float() @ w32.t()
        err = (y.float() - ref).abs().max().item()
        assert err <= 2e-3 * ref.abs().max().item(), (M, err)
    del w32


@pytest.mark.parametrize("N,K", [(128, 128), (264, 400), (6144, 2112), (100, 36), (7, 1000)])
def test_quantize_matches_oracle(ops, dev, N, K):
    """Device quantizer == the oracle restatement of _sm70_attn_fp8_quantize,
    bit for bit (codes and scales), including partial edge blocks, an
    all-zero block (scale floor 1e-12) and saturating outliers."""
    g = torch.Generator().manual_seed(N * 31 + K)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.float16)
    w[: min(N, 128), : min(K, 128)] = 0  # a zero block
    if N > 130 and K > 130:
        w[130, 131] = 60000.0  # outlier: its block's scale follows it
        w[131, 130] = -3e-7     # fp16 denormal
    q, s = ops._sm70_attn_fp8_quantize(w.to(dev))
    rq, rs = O.attn_fp8_quantize(w)
    assert torch.equal(s.cpu(), rs)
    assert torch.equal(q.cpu(), rq)
