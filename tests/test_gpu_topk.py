"""GPU parity: decode top-k and the prefill row top-k (persistent_topk),
bit-exact against the C oracle on identical score tensors (ties, -inf,
seq_len <= k, all-equal rows, inconsistent histogram)."""
import pytest
import torch

from oracle import cref
from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu


def hist_of(score, seq):
    B, W = score.shape
    h = torch.zeros(B, 4096, dtype=torch.int32)
    for b in range(B):
        L = min(int(seq[b]), W)
        h[b] = torch.bincount((O.mono_key(score[b, :L]) >> 20).long(), minlength=4096).to(torch.int32)
    return h


def scores(kind, B, W, g):
    if kind == "randn":
        return torch.randn(B, W, generator=g)
    if kind == "ties":
        return torch.round(torch.randn(B, W, generator=g) * 2) / 2
    if kind == "equal":
        return torch.full((B, W), 0.25)
    if kind == "narrow":  # one level-1 bin holds most keys: the select narrows on the row
        return 1.0 + torch.randn(B, W, generator=g) * 1e-3
    if kind == "rising":  # scores grow along the row: a first-chunk threshold estimate overflows
        return torch.arange(W).float().expand(B, W) * 1e-3 + torch.randn(B, W, generator=g)
    if kind == "falling":  # scores shrink along the row: the estimate lies above the threshold
        return -torch.arange(W).float().expand(B, W) * 1e-3 + torch.randn(B, W, generator=g)
    if kind == "mixed":
        s = torch.randn(B, W, generator=g) * 1e3
        s[:, ::3] = float("-inf")
        s[:, 1::7] = -0.0
        s[:, 2::7] = 0.0
        return s
    raise ValueError(kind)


CASES = [
    ("randn", 4, 65536, [65536, 65000, 3000, 2049]),
    ("ties", 3, 20000, [20000, 2048, 2047]),
    ("equal", 2, 10000, [10000, 5000]),
    ("mixed", 2, 33000, [33000, 16385]),
    ("randn", 1, 100, [100]),
    ("randn", 2, 70000, [0, 70000]),
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}-{c[1]}x{c[2]}" for c in CASES])
@pytest.mark.parametrize("K", [2048, 512, 1])
def test_decode_topk(ops, dev, case, K):
    kind, B, W, seq = case
    g = torch.Generator().manual_seed(B * W + K)
    s = scores(kind, B, W, g)
    seq = torch.tensor(seq, dtype=torch.int32)
    idx = torch.full((B, K), 123, dtype=torch.int32, device=dev)
    ops.sm70_decode_topk(idx, s.to(dev), seq.to(dev), hist_of(s, seq).to(dev), K)
    assert torch.equal(idx.cpu(), cref.topk_rows(s, seq, K))


def test_decode_topk_rebuilds_bad_hist(ops, dev):
    g = torch.Generator().manual_seed(5)
    s = torch.randn(2, 9000, generator=g)
    seq = torch.tensor([9000, 8000], dtype=torch.int32)
    idx = torch.empty(2, 2048, dtype=torch.int32, device=dev)
    ops.sm70_decode_topk(idx, s.to(dev), seq.to(dev), torch.zeros(2, 4096, dtype=torch.int32, device=dev), 2048)
    assert torch.equal(idx.cpu(), cref.topk_rows(s, seq, 2048))


@pytest.mark.parametrize("kind,B,W,seq,K", [
    ("equal", 1, 40000, [40000], 2048),       # candidate set above the LDS cap: whole-row path
    ("ties", 2, 50000, [50000, 30001], 2048),  # many keys share the threshold bin
    ("randn", 100, 5000, None, 256),            # more rows than the two-kernel path takes
    ("randn", 64, 20000, None, 2048),           # rows x 4096-key groups past one launch round: scan + select
    ("randn", 3, 3000, [2049, 2048, 3000], 2048),
])
def test_decode_topk_paths(ops, dev, kind, B, W, seq, K):
    """The decode top-k's scan/select path, its whole-row fallbacks and the
    one-workgroup-per-row path all give the exact selection."""
    g = torch.Generator().manual_seed(B * 7 + W)
    s = scores(kind, B, W, g)
    if seq is None:
        seq = [W - (i * 37) % 1000 for i in range(B)]
    seq = torch.tensor(seq, dtype=torch.int32)
    idx = torch.full((B, K), 123, dtype=torch.int32, device=dev)
    ops.sm70_decode_topk(idx, s.to(dev), seq.to(dev), hist_of(s, seq).to(dev), K)
    assert torch.equal(idx.cpu(), cref.topk_rows(s, seq, K))


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}-{c[1]}x{c[2]}" for c in CASES])
def test_persistent_topk(ops, dev, case):
    kind, B, W, seq = case
    g = torch.Generator().manual_seed(B + W)
    s = scores(kind, B, W, g)
    seq = torch.tensor(seq, dtype=torch.int32)
    out = torch.full((B, 2048), 77, dtype=torch.int32, device=dev)
    ws = torch.empty(1 << 20, dtype=torch.uint8, device=dev)
    ops.persistent_topk(s.to(dev), seq.view(B, 1).to(dev), out, ws, 2048, W)
    assert torch.equal(out.cpu(), cref.topk_rows(s, seq, 2048))


WIDE_CASES = [
    ("narrow", 2, 40000, [40000, 39000]),   # level-1 bin over the LDS list: a 10-bit row pass first
    ("equal", 1, 30000, [30000]),           # ties down to the last digit: bitmap of ties from the row
    ("randn", 2, 184320, [184320, 100000]),  # wide rows: one workgroup per CU, larger list
    ("ties", 1, 600000, [600000]),          # bitmaps past the LDS budget: three-read kernel
    ("randn", 2, 30001, [30001, 29998]),    # row stride not a multiple of 4: 4-byte loads
    ("rising", 2, 50000, [50000, 30000]),   # candidate estimate overflows: second read
    ("falling", 2, 50000, [50000, 30000]),  # estimate above the threshold bin: second read
]


@pytest.mark.parametrize("case", WIDE_CASES, ids=[f"{c[0]}-{c[1]}x{c[2]}" for c in WIDE_CASES])
def test_persistent_topk_select_paths(ops, dev, case):
    """Every branch of the whole-row select: list overflow narrowed on the
    row, all-tied rows, wide rows and the fallback for very wide rows."""
    kind, B, W, seq = case
    g = torch.Generator().manual_seed(3 * B + W)
    s = scores(kind, B, W, g)
    seq = torch.tensor(seq, dtype=torch.int32)
    out = torch.full((B, 2048), 77, dtype=torch.int32, device=dev)
    ws = torch.empty(1 << 20, dtype=torch.uint8, device=dev)
    ops.persistent_topk(s.to(dev), seq.view(B, 1).to(dev), out, ws, 2048, W)
    assert torch.equal(out.cpu(), cref.topk_rows(s, seq, 2048))


def _decode_topk_abi(pkg, idx, s, seq, h, K, ws, stream=None):
    st = stream if stream is not None else torch.cuda.current_stream()
    pkg._lib.call("mi355_dsa_decode_topk", idx.data_ptr(), s.data_ptr(), seq.data_ptr(),
                  h.data_ptr(), s.size(0), s.size(1), K, ws.data_ptr(), ws.numel(), st.cuda_stream)


def test_decode_topk_one_launch_workspace(pkg, dev):
    """The one-launch decode top-k keeps no state in its workspace (its
    arrival counters live in the library's per-device pool): a workspace
    holding arbitrary bytes, one reused across calls of other shapes and bad
    histograms, and calls on two streams at once (each stream its own
    counter slot) all give the exact selection."""
    L = pkg._lib.lib()
    g = torch.Generator().manual_seed(77)
    calls = [
        ("randn", 4, 65536, [65536, 60000, 3000, 2049], 2048, False),
        ("ties", 2, 9000, [9000, 8000], 512, False),
        ("narrow", 3, 20000, [20000, 19000, 100], 2048, True),   # bad histogram: whole row
        ("randn", 4, 65536, [65536] * 4, 2048, False),
        ("mixed", 1, 184320, [184320], 2048, False),
    ]
    wsb = max(L.mi355_dsa_decode_topk_workspace_size(B, W, K) for _, B, W, _, K, _ in calls)
    for fill in (0xFF, None):
        ws = (torch.full((wsb,), fill, dtype=torch.uint8, device=dev) if fill is not None
              else torch.randint(0, 256, (wsb,), dtype=torch.uint8, device=dev))
        for kind, B, W, seq, K, bad in calls:
            s = scores(kind, B, W, g)
            seq_t = torch.tensor(seq, dtype=torch.int32)
            h = hist_of(s, seq_t)
            if bad:
                h[0] = 0
            idx = torch.full((B, K), 123, dtype=torch.int32, device=dev)
            _decode_topk_abi(pkg, idx, s.to(dev), seq_t.to(dev), h.to(dev), K, ws)
            assert torch.equal(idx.cpu(), cref.topk_rows(s, seq_t, K)), (fill, kind, B, W)
    # two streams, each with its own workspace, launched back to back
    st = [torch.cuda.Stream(), torch.cuda.Stream()]
    jobs = []
    for i in range(2):
        s = scores("randn", 4, 65536, g)
        seq_t = torch.tensor([65536, 65000 - i, 40000, 2100], dtype=torch.int32)
        jobs.append((s, seq_t, s.to(dev), seq_t.to(dev), hist_of(s, seq_t).to(dev),
                     torch.empty(4, 2048, dtype=torch.int32, device=dev),
                     torch.empty(wsb, dtype=torch.uint8, device=dev)))
    torch.cuda.synchronize()
    for i, (_, _, sd, qd, hd, idx, ws) in enumerate(jobs):
        _decode_topk_abi(pkg, idx, sd, qd, hd, 2048, ws, stream=st[i])
    torch.cuda.synchronize()
    for s, seq_t, _, _, _, idx, _ in jobs:
        assert torch.equal(idx.cpu(), cref.topk_rows(s, seq_t, 2048))


def test_decode_topk_one_launch_graph_replays(pkg, dev):
    """One-launch decode top-k captured in a HIP graph: every replay, with the
    scores and histograms rewritten in place between replays and an eager
    call on the same workspace in between, equals the oracle (each row's
    last workgroup leaves its arrival counter zero)."""
    L = pkg._lib.lib()
    B, W, K = 4, 65536, 2048
    seq = torch.tensor([65536, 50000, 2049, 30000], dtype=torch.int32)
    g = torch.Generator().manual_seed(78)
    wsb = L.mi355_dsa_decode_topk_workspace_size(B, W, K)
    sd = torch.empty(B, W, device=dev)
    hd = torch.empty(B, 4096, dtype=torch.int32, device=dev)
    qd = seq.to(dev)
    idx = torch.empty(B, K, dtype=torch.int32, device=dev)
    ws = torch.full((wsb,), 0x5A, dtype=torch.uint8, device=dev)
    s = scores("randn", B, W, g)
    sd.copy_(s)
    hd.copy_(hist_of(s, seq))
    _decode_topk_abi(pkg, idx, sd, qd, hd, K, ws)  # eager first call, outside capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _decode_topk_abi(pkg, idx, sd, qd, hd, K, ws)
    for i, kind in enumerate(["ties", "randn", "mixed"]):
        s = scores(kind, B, W, g)
        sd.copy_(s)
        hd.copy_(hist_of(s, seq))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(idx.cpu(), cref.topk_rows(s, seq, K)), f"replay {i}"
        other = torch.empty_like(idx)
        _decode_topk_abi(pkg, other, sd, qd, hd, K, ws)  # eager, same workspace
        torch.cuda.synchronize()
        assert torch.equal(other, idx), f"eager after replay {i}"
    del graph


MANY_ROW_CASES = [
    ("randn", 600, 8192, "causal"),     # lengths crossing k (rows <= k select everything)
    ("randn", 1024, 20001, "full"),     # row stride not a multiple of 4: 4-byte loads
    ("ties", 530, 6000, "full"),
    ("equal", 512, 5000, "full"),       # one level-1 bin: ties down to the last digit
    ("equal", 520, 20000, "full"),      # every list overflows: rows selected again
    ("alternate", 700, 12000, "full"),  # neighbouring rows 100x apart in scale
    ("rising", 600, 12000, "full"),
    ("mixed", 777, 9000, "ragged"),     # lengths from 0 to the width
]


@pytest.mark.parametrize("case", MANY_ROW_CASES, ids=[f"{c[0]}-{c[1]}x{c[2]}-{c[3]}" for c in MANY_ROW_CASES])
def test_persistent_topk_many_rows(ops, dev, case):
    """Calls of more rows than CUs, several workgroups per CU: every branch
    (candidate list within bounds, list overflow re-selected by the whole
    workgroup, ties, rows of length <= k, ragged lengths) gives the exact
    selection."""
    kind, R, W, lens = case
    g = torch.Generator().manual_seed(R * 3 + W)
    if kind == "alternate":
        s = torch.randn(R, W, generator=g) * (1.0 + 99.0 * (torch.arange(R) % 2)).view(R, 1)
    else:
        s = scores(kind, R, W, g)
    if lens == "causal":
        seq = torch.clamp(torch.arange(R) + (W - R + 1), min=1)
    elif lens == "full":
        seq = torch.full((R,), W)
    else:
        seq = torch.randint(0, W + 1, (R,), generator=g)
    seq = seq.to(torch.int32)
    out = torch.full((R, 2048), 77, dtype=torch.int32, device=dev)
    ws = torch.empty(1 << 20, dtype=torch.uint8, device=dev)
    ops.persistent_topk(s.to(dev), seq.view(R, 1).to(dev), out, ws, 2048, W)
    assert torch.equal(out.cpu(), cref.topk_rows(s, seq, 2048))


def test_decode_topk_many_rows_bad_hist(ops, dev):
    """More rows than the two-kernel path takes, with histograms that do not
    count the rows: each row's histogram is rebuilt from its scores."""
    g = torch.Generator().manual_seed(21)
    B, W = 80, 6000
    s = scores("narrow", B, W, g)
    seq = torch.tensor([W - 13 * i for i in range(B)], dtype=torch.int32)
    h = hist_of(s, seq)
    h[::2] = 0
    idx = torch.empty(B, 2048, dtype=torch.int32, device=dev)
    ops.sm70_decode_topk(idx, s.to(dev), seq.to(dev), h.to(dev), 2048)
    assert torch.equal(idx.cpu(), cref.topk_rows(s, seq, 2048))


def test_persistent_topk_causal_block(ops, dev):
    """A 128-row prefill sub-block with causal lengths (rows < 2048 select
    everything up to themselves)."""
    g = torch.Generator().manual_seed(9)
    R, W = 128, 4096
    s = torch.randn(R, W, generator=g)
    seq = torch.arange(1985, 1985 + R, dtype=torch.int32) * 2 - 1985  # crosses 2048
    out = torch.empty(R, 2048, dtype=torch.int32, device=dev)
    ops.persistent_topk(s.to(dev), seq.view(R, 1).to(dev), out,
                        torch.empty(1 << 20, dtype=torch.uint8, device=dev), 2048, W)
    assert torch.equal(out.cpu(), cref.topk_rows(s, seq, 2048))


def _random_cases(n=16, seed=1234):
    """Deterministic random shapes for the decode top-k: row counts on both
    sides of the two-kernel limit, widths up to 180k, K from 1 to 4095,
    seq_len from 0 to the width, every score kind above."""
    import random
    rng = random.Random(seed)
    kinds = ["randn", "ties", "equal", "narrow", "rising", "falling", "mixed"]
    out = []
    for i in range(n):
        kind = rng.choice(kinds)
        B = rng.choice([1, 2, 3, 4, 7, 16, 33, 64, 65])
        W = rng.choice([2100, 4096, 9000, 20000, 65536, 184320])
        while B * W > 3_000_000:
            B = max(1, B // 2)
        K = rng.choice([1, 7, 100, 512, 2047, 2048, 4095])
        seq = [rng.choice([W, W - rng.randrange(0, max(1, W // 2)), rng.randrange(0, W + 1)])
               for _ in range(B)]
        out.append((i, kind, B, W, K, seq))
    return out


@pytest.mark.parametrize("case", _random_cases(), ids=lambda c: f"r{c[0]}-{c[1]}-{c[2]}x{c[3]}-k{c[4]}")
def test_decode_topk_random_shapes(ops, dev, case):
    """Randomised shapes and lengths, bit-exact against the C oracle."""
    i, kind, B, W, K, seq = case
    g = torch.Generator().manual_seed(1000 + i)
    s = scores(kind, B, W, g)
    seq = torch.tensor(seq, dtype=torch.int32)
    idx = torch.full((B, K), 123, dtype=torch.int32, device=dev)
    ops.sm70_decode_topk(idx, s.to(dev), seq.to(dev), hist_of(s, seq).to(dev), K)
    assert torch.equal(idx.cpu(), cref.topk_rows(s, seq, K))
