"""GPU parity: the MLA latent cache writer (concat_and_cache_mla, "auto" and
"fp8_ds_mla"), bit-exact against the oracle (oracle/dsa_oracle.py
concat_and_cache_mla) for fp16 and bf16 inputs, and read back by the sparse
MLA kernel."""
import pytest
import torch

from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu


def _run(pkg, dev, kv, kv_c, k_pe, slot, dtype):
    kd = kv.to(dev)
    pkg._cache_ops.concat_and_cache_mla(kv_c.to(dev), k_pe.to(dev), kd, slot.to(dev), dtype,
                                        torch.ones((), device=dev))
    return kd.cpu()


@pytest.mark.parametrize("T,in_dtype,slot_dtype", [
    (1, torch.float16, torch.int64), (300, torch.float16, torch.int32),
    (300, torch.bfloat16, torch.int64), (65536, torch.float16, torch.int64),
    (65536, torch.bfloat16, torch.int32)])
def test_fp8_ds_mla_bitexact(pkg, dev, T, in_dtype, slot_dtype):
    g = torch.Generator().manual_seed(T)
    page = 64
    nblk = (T + page - 1) // page + 2
    kv_c = torch.randn(T + 5, 512, generator=g) * torch.rand(T + 5, 1, generator=g) * 4
    kv_c[1::11] *= 1e-4   # small tiles: denormal codes
    kv_c[2::13, 128:256] = 0.0  # a zero tile: FLT_MIN scale
    kv_c = kv_c.to(in_dtype)
    k_pe = torch.randn(T + 5, 64, generator=g).to(in_dtype)
    slot = torch.randperm(nblk * page, generator=g)[:T].to(slot_dtype)
    slot[::17] = -1
    kv = torch.randint(0, 256, (nblk, page, 656), generator=g, dtype=torch.int32).to(torch.uint8)
    got = _run(pkg, dev, kv, kv_c, k_pe, slot, "fp8_ds_mla")
    assert torch.equal(got, O.concat_and_cache_mla(kv, kv_c, k_pe, slot, "fp8_ds_mla"))


def test_fp8_ds_mla_known_rows(pkg, dev):
    x = torch.zeros(3, 512)
    x[:, 0] = 448.0
    x[0, 1:7] = torch.tensor([1.0625, 1.1875, 2.0 ** -10, 3 * 2.0 ** -10, -448.0, 240.0])
    x[0, 7] = -0.0
    x[1, 128] = 65504.0
    x[1, 129:256] = torch.linspace(-65000, 65000, 127)
    x[2, 256:384] = torch.linspace(-447, 447, 128)
    for dt in (torch.float16, torch.bfloat16):
        kv_c = x.to(dt)
        k_pe = torch.randn(3, 64).to(dt)
        kv = torch.zeros(1, 4, 656, dtype=torch.uint8)
        slot = torch.tensor([3, 0, 1])
        got = _run(pkg, dev, kv, kv_c, k_pe, slot, "fp8_ds_mla")
        assert torch.equal(got, O.concat_and_cache_mla(kv, kv_c, k_pe, slot, "fp8_ds_mla"))
        assert got.view(-1, 656)[3, 7].item() == 0x80  # -0 keeps its sign


def test_strided_views_and_auto_dtype(pkg, dev):
    g = torch.Generator().manual_seed(5)
    T = 257
    kv = torch.randn(T, 576, generator=g).half()          # [kv_c | k_pe] of one projection
    kv_c, k_pe = kv[:, :512], kv[:, 512:]                  # row stride 576 for both
    slot = torch.randperm(5 * 64, generator=g)[:T]
    cache8 = torch.zeros(5, 64, 656, dtype=torch.uint8)
    d8 = cache8.to(dev)
    kd = kv.to(dev)
    pkg._cache_ops.concat_and_cache_mla(kd[:, :512], kd[:, 512:], d8, slot.to(dev),
                                        "fp8_ds_mla", torch.ones((), device=dev))
    assert torch.equal(d8.cpu(), O.concat_and_cache_mla(cache8, kv_c, k_pe, slot, "fp8_ds_mla"))
    cache16 = torch.zeros(5, 64, 576, dtype=torch.float16)
    d16 = cache16.to(dev)
    pkg._cache_ops.concat_and_cache_mla(kd[:, :512], kd[:, 512:], d16, slot.to(dev), "auto",
                                        torch.ones((), device=dev))
    assert torch.equal(d16.cpu(), O.concat_and_cache_mla(cache16, kv_c, k_pe, slot, "auto"))


def test_written_cache_read_by_sparse_mla(pkg, dev):
    """Rows written by the writer are read back by the sparse MLA decode
    kernel: its output equals the oracle attention over the same cache."""
    g = torch.Generator().manual_seed(9)
    B, H, page, nblk, ctx = 2, 64, 64, 40, 2300
    n = nblk * page
    lat = torch.randn(n, 576, generator=g) / 24.0
    slot = torch.randperm(n, generator=g)
    cache = torch.zeros(nblk, page, 656, dtype=torch.uint8, device=dev)
    pkg._cache_ops.concat_and_cache_mla(lat[:, :512].half().to(dev), lat[:, 512:].half().to(dev),
                                        cache, slot.to(dev), "fp8_ds_mla",
                                        torch.ones((), device=dev))
    mb = (ctx + page - 1) // page
    bt = torch.stack([torch.randperm(nblk, generator=g)[:mb] for _ in range(B)]).to(torch.int32)
    seq = torch.tensor([ctx, 1500], dtype=torch.int32)
    idx = torch.full((B, 2048), -1, dtype=torch.int32)
    for b in range(B):
        sel = torch.randperm(int(seq[b]), generator=g)[:2048].sort().values
        idx[b, :sel.numel()] = sel.to(torch.int32)
    q = (torch.randn(B, H, 576, generator=g) / 4).half()
    o = torch.empty(B, H, 512, dtype=torch.float16, device=dev)
    lse = torch.empty(B, H, device=dev)
    pkg._sm70_ops.sm70_sparse_mla_decode(o, lse, q.to(dev), cache, idx.to(dev), bt.to(dev),
                                         seq.to(dev), 576 ** -0.5)
    ro, rl = O.sparse_mla(q, cache.cpu(), idx, bt, seq, 576 ** -0.5)
    torch.testing.assert_close(o.float().cpu(), ro, rtol=2e-3, atol=1e-3)
    assert (lse.cpu() - rl).abs().max().item() <= 1e-4
