"""GPU parity of the per-head projection kernel (mi355_dsa_head_proj) that
replaces the layer's q_nope @ W_UK_T + concat(q_pe) and o @ W_UV bmms
(reference/triton_mla.py:388-418, :486-492).

Dyadic inputs make every product and sum exact in fp32, so the kernel must
equal the fp64 oracle bit for bit; on random inputs it must be within the
fp16 rounding of the output (2^-11 relative) plus the fp32 accumulation
error (1e-4 of the output scale), and within the same bound of torch.bmm."""
import pytest
import torch

from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu


def weights(pkg, dev, g, H, P, V, dyadic):
    if dyadic:
        uk = (torch.randint(-4, 5, (H, P, 512), generator=g) / 16).to(torch.float16)
        uv = (torch.randint(-4, 5, (H, 512, V), generator=g) / 16).to(torch.float16)
    else:
        uk = (torch.randn(H, P, 512, generator=g) / P ** 0.5).to(torch.float16)
        uv = (torch.randn(H, 512, V, generator=g) / 512 ** 0.5).to(torch.float16)
    return pkg.dsa_layer.DsaLayerWeights(uk.to(dev), uv.to(dev), 0.1), uk, uv


def close(got, want):
    err = (got.double() - want).abs()
    bound = 2.0 ** -11 * want.abs() + 1e-4 * want.abs().max() + 1e-6
    assert torch.all(err <= bound), err.max().item()


SHAPES = [  # T, H, P, V
    (4, 64, 128, 128),
    (1, 64, 128, 128),
    (17, 16, 192, 256),     # partial token tile, GLM-sized nope / v dims
    (3000, 8, 128, 128),    # several token chunks (the wide many-token kernel)
    (1000, 8, 256, 256),    # wide kernel with K split over two waves per column group
    (1500, 16, 128, 128),
    (2, 128, 64, 512),      # small K, wide V
]


@pytest.mark.parametrize("shape", SHAPES, ids=[f"T{s[0]}H{s[1]}P{s[2]}V{s[3]}" for s in SHAPES])
@pytest.mark.parametrize("dyadic", [True, False], ids=["exact", "random"])
def test_q_latent_and_v_up(pkg, dev, shape, dyadic):
    T, H, P, V = shape
    g = torch.Generator().manual_seed(T * 7 + H + P + V + int(dyadic))
    w, uk, uv = weights(pkg, dev, g, H, P, V, dyadic)
    if dyadic:
        q = (torch.randint(-4, 5, (T, H, P + 64), generator=g) / 8).to(torch.float16)
        o = (torch.randint(-4, 5, (T, H, 512), generator=g) / 8).to(torch.float16)
    else:
        q = torch.randn(T, H, P + 64, generator=g).to(torch.float16)
        o = (torch.randn(T, H, 512, generator=g) / 4).to(torch.float16)
    m = pkg.dsa_layer
    ql = m.q_latent(q.to(dev), w).cpu()
    out = m.v_up(o.to(dev), w).cpu()
    want_ql = O.q_latent(q, uk)
    want_out = O.v_up(o, uv)
    assert torch.equal(ql[..., 512:], q[..., P:])  # q_pe carried unchanged
    if dyadic:
        assert torch.equal(ql, want_ql.to(torch.float16))
        assert torch.equal(out, want_out.to(torch.float16))
    else:
        exact_ql = torch.einsum("thp,hpl->thl", q[..., :P].double(), uk.double())
        close(ql[..., :512].float(), exact_ql)
        close(out.float(), want_out.double())
        # and the reference's own bmm formulation, computed on the GPU in fp32
        qn = q[..., :P].to(dev).float().transpose(0, 1).contiguous()
        bm = torch.bmm(qn, uk.to(dev).float()).transpose(0, 1).cpu()
        close(ql[..., :512].float(), bm.double())


def test_strided_inputs(pkg, dev):
    """q as a slice of a wider tensor (head stride 256), o as a head slice."""
    T, H, P, V = 5, 16, 128, 128
    g = torch.Generator().manual_seed(3)
    w, uk, uv = weights(pkg, dev, g, H, P, V, True)
    big = (torch.randint(-4, 5, (T, H, 256), generator=g) / 8).to(torch.float16)
    q = big[:, :, :P + 64]
    ob = (torch.randint(-4, 5, (T, 2 * H, 512), generator=g) / 8).to(torch.float16)
    o = ob[:, 1::2]
    m = pkg.dsa_layer
    ql = m.q_latent(big.to(dev)[:, :, :P + 64], w).cpu()
    out = m.v_up(ob.to(dev)[:, 1::2], w).cpu()
    assert torch.equal(ql, O.q_latent(q, uk).to(torch.float16))
    assert torch.equal(out, O.v_up(o.contiguous(), uv).to(torch.float16))


def test_every_token_written(pkg, dev):
    """Outputs start as NaN; every element of [T, H, 576] / [T, H*V] must be
    overwritten (no token or column left out at tile / chunk edges)."""
    T, H, P, V = 2049, 4, 128, 128
    g = torch.Generator().manual_seed(5)
    w, uk, uv = weights(pkg, dev, g, H, P, V, True)
    q = (torch.randint(-4, 5, (T, H, P + 64), generator=g) / 8).to(torch.float16).to(dev)
    out = torch.full((T, H, 576), float("nan"), dtype=torch.float16, device=dev)
    pkg.dsa_layer.head_proj(out, q, w.uk_t, 64)
    assert not torch.isnan(out).any()
    assert torch.equal(out.cpu(), O.q_latent(q.cpu(), uk).to(torch.float16))
