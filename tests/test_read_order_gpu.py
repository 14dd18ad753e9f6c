"""GPU checks of the read's token order (C ABI naylis_mom_read_order) against
a CPU statement of its rule: for top-2 routing over at most 32 blocks, the
tokens of the whole batch stably sorted by their block pair, kept only when
that lowers the number of (128-token tile, block) pairs by at least 10 %;
sequence order otherwise (and for every other routing)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def cpu_order(top_idx, E):
    idx = top_idx.reshape(-1, top_idx.shape[-1]).numpy().astype(np.int64)
    N, k = idx.shape
    ident = np.arange(N)
    if k != 2 or E > 32:
        return ident, None
    a = np.clip(idx[:, 0], 0, E - 1)
    b = np.clip(idx[:, 1], 0, E - 1)
    key = np.minimum(a, b) * E + np.maximum(a, b)
    srt = np.argsort(key, kind="stable")

    def pairs(order):
        tot = 0
        for t0 in range(0, N, 128):
            sel = idx[order[t0:t0 + 128]]
            tot += len(np.unique(sel[(sel >= 0) & (sel < E)]))
        return tot

    return (srt if pairs(srt) * 10 <= pairs(ident) * 9 else ident), key


def gpu_order(top_idx, E, dev):
    from naylis_amd import _lib
    lib = _lib.load()
    B, S, k = top_idx.shape
    ti = top_idx.to(torch.int32).to(dev).contiguous()
    order = torch.full((1 + B * S,), -7, dtype=torch.int32, device=dev)
    ws = torch.empty(lib.naylis_mom_read_order_workspace_bytes(B, S, E, k), dtype=torch.uint8, device=dev)
    _lib.check(lib.naylis_mom_read_order(ti.data_ptr(), order.data_ptr(), ws.data_ptr(), ws.numel(), B, S, E, k,
                                         torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    buf = order.cpu().numpy()
    assert buf[0] in (0, 1), "mode word"
    return buf[1:] if buf[0] == 1 else np.arange(B * S)


@pytest.mark.parametrize("B,S,E,k,coherent", [
    (8, 2048, 8, 2, False),    # config 2 geometry, incoherent routing: grouping pays
    (4, 4096, 32, 2, True),    # config 4 style: one block set per 128-token tile, sequence order kept
    (4, 4096, 32, 2, False),   # 32 blocks, incoherent: hundreds of keys, many of them empty
    (2, 300, 8, 2, False),     # ragged token count
    (2, 300, 8, 3, False),     # top-3: sequence order
    (1, 1000, 64, 2, False),   # more than 32 blocks: sequence order
    (3, 129, 4, 1, False),     # top-1: sequence order
])
def test_read_order_matches_cpu_rule(B, S, E, k, coherent, dev):
    g = torch.Generator().manual_seed(B * S + E)
    if coherent:
        idx = torch.empty(B, S, k, dtype=torch.int64)
        for b in range(B):
            for t0 in range(0, S, 128):
                blocks = torch.randperm(E, generator=g)[:4]
                n = min(128, S - t0)
                pick = torch.stack([torch.randperm(4, generator=g)[:k] for _ in range(n)])
                idx[b, t0:t0 + n] = blocks[pick]
    else:
        idx = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(B * S)]).view(B, S, k)
    want, _ = cpu_order(idx, E)
    got = gpu_order(idx, E, dev)
    assert np.array_equal(np.sort(got), np.arange(B * S)), "not a permutation"
    assert np.array_equal(got, want)
    if coherent:
        assert np.array_equal(got, np.arange(B * S))
    elif E <= 32 and k == 2 and B * S > 1024:
        assert not np.array_equal(got, np.arange(B * S)), "grouping should pay for incoherent routing"


@pytest.mark.parametrize("pairs", [[(3, 3)], [(3, 3), (5, 1), (1, 5), (0, 7)]])
def test_read_order_repeated_pairs(pairs, dev):
    """Few keys with long segments (one key covering every tile), and a
    duplicated id (both selections naming one block)."""
    g = torch.Generator().manual_seed(len(pairs))
    B, S, E = 2, 3000, 8
    pick = torch.randint(0, len(pairs), (B, S), generator=g)
    idx = torch.tensor(pairs, dtype=torch.int64)[pick]
    want, _ = cpu_order(idx, E)
    got = gpu_order(idx, E, dev)
    assert np.array_equal(got, want)
