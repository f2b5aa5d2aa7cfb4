"""Oracle of the MLA latent cache writer (vLLM concat_and_cache_mla,
"auto" and "fp8_ds_mla"), pinned by known answers, an independent
restatement (dsmla_rows with per-tile scales) and a round-trip bound.
The upstream kernel is not in the reference (only its amax fix,
patches/glm5-v100-sm70-glue.patch:517-531), so beyond these checks its
parity is unpinned."""
import numpy as np
import torch

from oracle import dsa_oracle as O

FLT_MIN = float(np.finfo(np.float32).tiny)


def rows(cache):
    return cache.view(-1, 656)


def test_tile_scales_ties_saturation_and_zero_tile():
    x = torch.zeros(1, 512)
    x[0, 0] = 448.0                       # tile 0: amax 448 -> scale 1
    x[0, 1:6] = torch.tensor([1.0625, 1.1875, -1.0625, 2.0 ** -10, 3 * 2.0 ** -10])
    x[0, 128] = -2.0                      # tile 1: amax 2 -> scale 2/448
    x[0, 129] = 1.0
    # tile 2 stays zero -> FLT_MIN scale; tile 3: amax 65504 (fp16 max)
    x[0, 384] = 65504.0
    x[0, 385] = -65504.0
    pe = torch.arange(64, dtype=torch.float16)[None]
    out = O.concat_and_cache_mla(torch.zeros(1, 4, 656, dtype=torch.uint8), x.half(), pe,
                                 torch.tensor([2]), "fp8_ds_mla")
    r = rows(out)[2]
    sc = r[512:528].view(torch.float32)
    assert sc[0].item() == 1.0
    assert sc[1].item() == np.float32(np.float32(2.0) / np.float32(448.0))
    assert sc[2].item() == FLT_MIN
    assert sc[3].item() == np.float32(np.float32(65504.0) / np.float32(448.0))
    # e4m3 codes: 448 -> 0x7e; RNE ties 1.0625 -> 1.0 (0x38), 1.1875 -> 1.25 (0x3a);
    # denormals 2^-10 -> 0 (tie to even), 3*2^-10 -> 2^-9 * 2 (0x02)
    assert r[:6].tolist() == [0x7E, 0x38, 0x3A, 0xB8, 0x00, 0x02]
    assert r[128].item() == 0xFE and r[129].item() == 0x76  # -448 and 224 = 1.75 * 2^7
    assert r[384].item() == 0x7E and r[385].item() == 0xFE
    assert bool((r[256:384] == 0).all())
    assert torch.equal(r[528:].view(torch.float16), pe[0])
    assert bool((rows(out)[[0, 1, 3]] == 0).all())


def test_matches_per_tile_dsmla_rows_and_skips_slots():
    g = torch.Generator().manual_seed(0)
    T = 50
    kv_c = (torch.randn(T, 512, generator=g) * torch.rand(T, 1, generator=g) * 3).half()
    k_pe = torch.randn(T, 64, generator=g).half()
    slot = torch.randperm(64 * 4, generator=g)[:T]
    slot[::7] = -1
    slot[3] = 10 ** 6
    out = O.concat_and_cache_mla(torch.zeros(4, 64, 656, dtype=torch.uint8), kv_c, k_pe, slot,
                                 "fp8_ds_mla")
    want = O.dsmla_rows(torch.cat([kv_c.float(), k_pe.float()], 1), per_tile=True)
    ok = (slot >= 0) & (slot < 256)
    assert torch.equal(rows(out)[slot[ok]], want[ok])
    mask = torch.ones(256, dtype=torch.bool)
    mask[slot[ok]] = False
    assert bool((rows(out)[mask] == 0).all())


def test_round_trip_bound_and_bf16_rope_bits():
    g = torch.Generator().manual_seed(1)
    T = 20
    kv_c = (torch.randn(T, 512, generator=g) * 5).to(torch.bfloat16)
    k_pe = torch.randn(T, 64, generator=g).to(torch.bfloat16)
    out = O.concat_and_cache_mla(torch.zeros(1, 32, 656, dtype=torch.uint8), kv_c, k_pe,
                                 torch.arange(T), "fp8_ds_mla")
    r = rows(out)[:T]
    assert torch.equal(r[:, 528:].contiguous().view(torch.bfloat16), k_pe)
    sc = r[:, 512:528].contiguous().view(torch.float32)
    deq = O.e4m3_decode(r[:, :512].contiguous()).view(T, 4, 128) * sc[:, :, None]
    x = kv_c.float().view(T, 4, 128)
    amax = x.abs().amax(dim=2, keepdim=True)
    # RNE to 3 mantissa bits: relative error <= 2^-4 of the value, absolute
    # error <= half the smallest subnormal step (2^-10 of the scale)
    err = (deq - x).abs()
    assert bool((err <= x.abs() / 16 + amax / 448 * 2.0 ** -10 + 1e-30).all())


def test_auto_dtype_concatenates():
    kv_c = torch.randn(3, 512).half()
    k_pe = torch.randn(3, 64).half()
    out = O.concat_and_cache_mla(torch.zeros(2, 2, 576, dtype=torch.float16), kv_c, k_pe,
                                 torch.tensor([3, -1, 0]), "auto")
    flat = out.view(-1, 576)
    assert torch.equal(flat[3], torch.cat([kv_c[0], k_pe[0]]))
    assert torch.equal(flat[0], torch.cat([kv_c[2], k_pe[2]]))
    assert bool((flat[1:3] == 0).all())
