"""GPU check of the allocation-free sparse MLA decode entry point
(mi355_dsa_sparse_mla_decode_noalloc, no counterpart in the reference: for
callers that cannot allocate device memory).  Called through the C ABI, its
outputs must equal mi355_dsa_sparse_mla_decode's (same kernels, caller
workspace) bit for bit: on two calls in a row, the second with a smaller
input, so the second call runs on a scratch array that still holds the
first call's partials.  A call whose split scratch exceeds the array's
maximum is rejected before any launch."""
import ctypes

import pytest
import torch

from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu

SCALE = 576 ** -0.5


def inputs(seed, B, H, ctx, topk, fp8, dev, nblk_extra=8, page=64):
    g = torch.Generator().manual_seed(seed)
    nblk = (ctx + page - 1) // page * B + nblk_extra
    lat = torch.randn(nblk * page, 576, generator=g)
    kv = (O.dsmla_rows(lat).view(nblk, page, 656) if fp8
          else lat.to(torch.float16).view(nblk, page, 576))
    mb = (ctx + page - 1) // page
    bt = torch.randperm(nblk, generator=g)[:B * mb].view(B, mb).to(torch.int32)
    idx = torch.stack([torch.randperm(ctx, generator=g)[:topk].sort().values
                       for _ in range(B)]).to(torch.int32)
    q = (torch.randn(B, H, 576, generator=g) * 0.05).to(torch.float16)
    seq = torch.full((B,), ctx, dtype=torch.int32)
    return [t.to(dev) for t in (q, kv, idx, bt, seq)]


def call(lib, noalloc, q, kv, idx, bt, seq):
    B, H = q.shape[:2]
    topk = idx.shape[1]
    fp8 = 1 if kv.dtype == torch.uint8 else 0
    o = torch.full((B, H, 512), float("nan"), dtype=torch.float16, device=q.device)
    lse = torch.full((B, H), float("nan"), device=q.device)
    st = torch.cuda.current_stream().cuda_stream
    n_rows = kv.numel() // kv.shape[-1]
    args = (o.data_ptr(), lse.data_ptr(), q.data_ptr(), B, H, kv.data_ptr(), fp8, n_rows,
            kv.shape[-2], idx.data_ptr(), topk, bt.data_ptr(), bt.shape[1], seq.data_ptr(),
            SCALE)
    if noalloc:
        rc = lib.mi355_dsa_sparse_mla_decode_noalloc(*args, st)
    else:
        need = lib.mi355_dsa_sparse_mla_workspace_size(B, H, topk)
        ws = torch.empty(max(need, 16), dtype=torch.uint8, device=q.device)
        rc = lib.mi355_dsa_sparse_mla_decode(*args, ws.data_ptr(), need, st)
        torch.cuda.synchronize()
        del ws
    assert rc == 0, lib.mi355_dsa_last_error()
    torch.cuda.synchronize()
    return o.cpu(), lse.cpu()


@pytest.mark.parametrize("fp8", [True, False], ids=["fp8", "fp16"])
def test_noalloc_equals_workspace_entry_point(lib, dev, fp8):
    # calls in a row, each needing less scratch than the one before: a 16-token
    # batch (64-head pipelined kernel, 16 key splits), C3's shape at a shorter
    # context (split decode), a small 16-head call
    for seed, B, H, ctx, topk in ((3, 16, 64, 3000, 2048), (1, 4, 64, 6000, 2048),
                                  (2, 2, 16, 900, 512)):
        ins = inputs(seed, B, H, ctx, topk, fp8, dev)
        o1, l1 = call(lib, True, *ins)
        o2, l2 = call(lib, False, *ins)
        assert torch.equal(o1.view(torch.int16), o2.view(torch.int16)), (seed, B, H)
        assert torch.equal(l1, l2), (seed, B, H)
        assert torch.isfinite(o1.float()).all()


def test_noalloc_rejects_oversize(lib, dev):
    cap = lib.mi355_dsa_sparse_mla_noalloc_max_bytes()
    assert cap == 32 << 20
    B, H, topk = 128, 16, 2048  # 16 splits of the 16-head split decode: 33.8 MB
    assert lib.mi355_dsa_sparse_mla_workspace_size(B, H, topk) > cap
    rc = lib.mi355_dsa_sparse_mla_decode_noalloc(None, None, None, B, H, None, 1, 0, 64, None,
                                                 topk, None, 1, None, SCALE, None)
    assert rc == 1
    assert b"maximum" in lib.mi355_dsa_last_error()
