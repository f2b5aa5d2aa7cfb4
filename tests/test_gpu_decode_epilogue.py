"""GPU check of mi355_dsa_decode_layer_attention, the decode layer's sparse
attention and W_UV projection: where the decode splits the keys (B <= 16, V
a multiple of 32) the split merge and the projection run as one launch.  Its
o, lse and out must equal, bit for bit, those of the two calls it replaces
(sm70_sparse_mla_decode, then the head projection as v_up), on the fused
shapes and on the shapes that take the two-call path (more tokens, no key
split, V not a multiple of 32, a padded or misaligned output).  The two
separate calls are pinned against the oracle by their own tests."""
import ctypes

import pytest
import torch

from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu

PAGE = 64

CASES = [
    # B, H, topk, fp8 cache, V, seq_lens (None: long contexts)
    (4, 64, 2048, True, 128, None),        # fp8 split decode (LDS-DMA gathers), fused
    (4, 64, 2048, False, 128, None),       # fp16 split decode, fused
    (12, 64, 2048, False, 128, None),      # pipelined kernel with a key split, fused
    (16, 16, 512, True, 64, None),         # 16 heads, 16 tokens, fused
    (5, 64, 2048, True, 128, [0, 1, 70, 3000, 5000]),  # empty / short rows, fused
    (20, 64, 2048, True, 128, None),       # B > 16: two calls
    (3, 64, 64, False, 128, None),         # no key split: two calls
    (4, 64, 2048, True, 48, None),         # V % 32 != 0: two calls
]


def _inputs(case, dev):
    B, H, topk, fp8, V, seqs = case
    g = torch.Generator().manual_seed(B * 131 + H + topk + V)
    seqs = seqs or [5000 + 37 * b for b in range(B)]
    nblk = max((max(seqs) + PAGE - 1) // PAGE, 1) + 4
    lat = torch.randn(nblk * PAGE, 576, generator=g) / 24.0
    kv = (O.dsmla_rows(lat).view(nblk, PAGE, 656) if fp8
          else lat.to(torch.float16).view(nblk, PAGE, 576))
    mb = max((max(seqs) + PAGE - 1) // PAGE, 1)
    bt = torch.stack([torch.randperm(nblk, generator=g)[:mb] for _ in range(B)]).to(torch.int32)
    idx = torch.full((B, topk), -1, dtype=torch.int32)
    for b, L in enumerate(seqs):
        n = min(L, topk)
        if n > 0:
            idx[b, :n] = torch.randperm(L, generator=g)[:n].sort().values.to(torch.int32)
    q = (torch.randn(B, H, 576, generator=g) / 4).to(torch.float16)
    W_UV = (torch.randn(H, 512, V, generator=g) / 24).to(torch.float16)
    sl = torch.tensor(seqs, dtype=torch.int32)
    return [t.to(dev) for t in (q, kv, idx, bt, sl, W_UV)]


def _weights(m, W_UV, dev):
    H = W_UV.shape[0]
    uk = torch.zeros(H, 128, 512, dtype=torch.float16, device=dev)
    return m.DsaLayerWeights(uk, W_UV, 576 ** -0.5)


def _separate(pkg, w, q, kv, idx, bt, sl):
    B, H = q.shape[:2]
    o = torch.full((B, H, 512), float("nan"), dtype=torch.float16, device=q.device)
    lse = torch.full((B, H), float("nan"), device=q.device)
    pkg._sm70_ops.sm70_sparse_mla_decode(o, lse, q, kv, idx, bt, sl, w.scale)
    return o, lse, pkg.dsa_layer.v_up(o, w)


def _bits(x):
    return x.view(torch.int16) if x.dtype == torch.float16 else x.view(torch.int32)


@pytest.mark.parametrize("case", CASES, ids=[f"B{c[0]}H{c[1]}k{c[2]}{'fp8' if c[3] else 'f16'}"
                                             f"V{c[4]}{'-short' if c[5] else ''}" for c in CASES])
def test_attention_equals_separate_calls(pkg, dev, case):
    m = pkg.dsa_layer
    q, kv, idx, bt, sl, W_UV = _inputs(case, dev)
    w = _weights(m, W_UV, dev)
    o1, lse1, out1 = _separate(pkg, w, q, kv, idx, bt, sl)
    L = m.DsaLayer(w, kv, torch.zeros(1, PAGE, 128, dtype=torch.float16, device=dev),
                   topk=idx.shape[1])
    o2, lse2, out2 = L._attention(q, idx, bt, sl)
    torch.cuda.synchronize()
    assert torch.equal(_bits(o1), _bits(o2))
    assert torch.equal(_bits(lse1), _bits(lse2))
    assert torch.equal(_bits(out1), _bits(out2))
    assert torch.isfinite(out2.float()).all()
    if case[5]:  # the empty row: lse -inf, o and out zero
        assert torch.isinf(lse2[0]).all() and not o2[0].any() and not out2[0].any()


@pytest.mark.parametrize("pad,offset", [(0, 0), (40, 0), (0, 1)],
                         ids=["dense", "padded-rows", "misaligned"])
def test_attention_output_layouts(pkg, lib, dev, pad, offset):
    """out rows `pad` elements longer than H * V, or the output base moved
    by one element (not 8-byte aligned: the two-call path)."""
    m = pkg.dsa_layer
    case = (4, 64, 2048, True, 128, None)
    q, kv, idx, bt, sl, W_UV = _inputs(case, dev)
    w = _weights(m, W_UV, dev)
    B, H, V = 4, 64, 128
    o1, lse1, out1 = _separate(pkg, w, q, kv, idx, bt, sl)
    st = H * V + pad
    buf = torch.full((B * st + offset + 8,), 7.0, dtype=torch.float16, device=dev)
    out = buf[offset:offset + B * st].view(B, st)
    o = torch.empty(B, H, 512, dtype=torch.float16, device=dev)
    lse = torch.empty(B, H, device=dev)
    ws_bytes = lib.mi355_dsa_sparse_mla_workspace_size(B, H, idx.shape[1])
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    rc = lib.mi355_dsa_decode_layer_attention(
        ctypes.c_void_p(out.data_ptr()), st, ctypes.c_void_p(o.data_ptr()),
        ctypes.c_void_p(lse.data_ptr()), ctypes.c_void_p(q.data_ptr()), B, H,
        ctypes.c_void_p(kv.data_ptr()), 1, kv.numel() // 656, PAGE,
        ctypes.c_void_p(idx.data_ptr()), idx.shape[1], ctypes.c_void_p(bt.data_ptr()),
        bt.shape[1], ctypes.c_void_p(sl.data_ptr()), ctypes.c_float(w.scale),
        ctypes.c_void_p(w.uv_t.data_ptr()), V, ctypes.c_void_p(ws.data_ptr()), ws_bytes,
        ctypes.c_void_p(stream))
    assert rc == 0, lib.mi355_dsa_last_error()
    torch.cuda.synchronize()
    assert torch.equal(_bits(o1), _bits(o)) and torch.equal(_bits(lse1), _bits(lse))
    assert torch.equal(_bits(out1), _bits(out[:, :H * V].contiguous()))
    if pad:
        assert (out[:, H * V:] == 7).all()
    assert (buf[:offset] == 7).all() and (buf[offset + B * st:] == 7).all()


def test_attention_rejects_short_rows(pkg, lib, dev):
    """An output row shorter than H * V is refused before any launch."""
    B, H, V = 2, 16, 64
    rc = lib.mi355_dsa_decode_layer_attention(
        ctypes.c_void_p(16), H * V - 4, ctypes.c_void_p(16), ctypes.c_void_p(16),
        ctypes.c_void_p(16), B, H, ctypes.c_void_p(16), 1, 64, PAGE, ctypes.c_void_p(16), 64,
        ctypes.c_void_p(16), 1, ctypes.c_void_p(16), ctypes.c_float(0.05), ctypes.c_void_p(16),
        V, None, 0, None)
    assert rc != 0
    assert b"n_head * V" in lib.mi355_dsa_last_error()
