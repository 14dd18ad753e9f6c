"""GPU checks of the read's token order (C ABI naylis_mom_read_order) against
a CPU statement of its rule: for top-2 routing over at most 32 blocks, the
tokens of the whole batch stably sorted by their block pair, kept only when
that lowers the number of (128-token tile, block) pairs by at least 10 %;
sequence order otherwise (and for every other routing).  For top-2 over at
most 32 blocks the buffer also carries the pair plan, checked against its own
CPU statement."""
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
    order = torch.full((int(lib.naylis_mom_read_order_words(B, S, E, k)),), -7, dtype=torch.int32, device=dev)
    ws = torch.empty(lib.naylis_mom_read_order_workspace_bytes(B, S, E, k), dtype=torch.uint8, device=dev)
    _lib.check(lib.naylis_mom_read_order(ti.data_ptr(), order.data_ptr(), ws.data_ptr(), ws.numel(), B, S, E, k,
                                         torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    buf = order.cpu().numpy()
    assert buf[0] in (0, 1), "mode word"
    if k == 2 and E <= 32:
        check_pair_plan(buf, top_idx, E)
    return buf[1:1 + B * S] if buf[0] == 1 else np.arange(B * S)


def check_pair_plan(buf, top_idx, E):
    """The pair plan after the order table (layout of read_common.h), against
    a CPU statement: the table is the stable sort by sorted block pair (also
    when the mode word keeps sequence order); the keys with tokens ascending,
    each with its blocks, first tile and tile count; each key's run cut into
    32-position tiles; forward items of up to 128 consecutive positions of a
    key (first position, token count and blocks)."""
    idx = top_idx.reshape(-1, 2).numpy().astype(np.int64)
    N = idx.shape[0]
    a = np.clip(idx[:, 0], 0, E - 1)
    b = np.clip(idx[:, 1], 0, E - 1)
    lo, hi = np.minimum(a, b), np.maximum(a, b)
    key = lo * E + hi
    srt = np.argsort(key, kind="stable")
    assert np.array_equal(buf[1:1 + N], srt), "grouped table"
    base = (1 + N + 3) // 4 * 4
    n_tiles, n_keys, n_fit = buf[base:base + 3]
    mk = min(E * (E + 1) // 2, N)
    max_tiles = (N + 31) // 32 + mk
    keys_off, tiles_off = base + 8, base + 8 + 4 * mk
    fit_off = tiles_off + 2 * max_tiles  # two words per forward item
    ukeys, counts = np.unique(key, return_counts=True)
    assert n_keys == len(ukeys)
    pos, t = 0, 0
    want_tiles, want_fit = [], []
    for kk, (uk, c) in enumerate(zip(ukeys, counts)):
        ka, kb, ts, nt = buf[keys_off + 4 * kk:keys_off + 4 * kk + 4]
        assert (ka, kb) == (uk // E, uk % E) and ts == t and nt == (c + 31) // 32, kk
        for j in range(nt):
            cnt = min(32, c - 32 * j)
            want_tiles.append((pos + 32 * j, cnt | (ka << 6) | (kb << 11) | (kk << 16)))
        for j in range(0, c, 128):
            want_fit.append((pos + j, min(128, c - j) | (ka << 16) | (kb << 21)))
        pos += c
        t += nt
    assert n_tiles == t and n_fit == len(want_fit)
    got_tiles = buf[tiles_off:tiles_off + 2 * t].reshape(-1, 2)
    assert np.array_equal(got_tiles, np.array(want_tiles).reshape(-1, 2)), "tiles"
    got_fit = buf[fit_off:fit_off + 2 * n_fit].reshape(-1, 2)
    assert np.array_equal(got_fit, np.array(want_fit).reshape(-1, 2)), "forward items"


@pytest.mark.parametrize("B,S,E,k,coherent", [
    (8, 2048, 8, 2, False),    # config 2 geometry, incoherent routing: grouping pays
    (4, 4096, 32, 2, True),    # config 4 style: one block set per 128-token tile, sequence order kept
    (4, 4096, 32, 2, False),   # 32 blocks, incoherent: hundreds of keys, many of them empty
    (2, 16384, 8, 2, False),   # 32 chunks of 1024 tokens
    (1, 20000, 32, 2, False),  # 32 blocks, a ragged last chunk
    (3, 4096, 32, 2, True),    # coherent, three sequences: sequence order kept
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
