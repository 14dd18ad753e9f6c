"""naylis_mom_read_bwd_noalloc (the read backward on the library's own
scratch array, no workspace argument, no allocation) against
naylis_mom_read_bwd with a caller workspace, through the C ABI: two calls in
a row, the second on a smaller read that finds the first one's contents in
the scratch array.  The read backward is deterministic (fixed-order
reductions), so the two entry points agree bitwise."""
import os
import re

import pytest
import torch

from naylis_amd import _lib

pytestmark = pytest.mark.gpu

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "naylis_mom.h")


def _max_bytes():
    m = re.search(r"#define NAYLIS_READ_BWD_NOALLOC_MAX_BYTES \(\(size_t\)(\d+) << (\d+)\)", open(HEADER).read())
    return int(m.group(1)) << int(m.group(2))


def _case(dev, B, S, H, HD, E, BS, K, seed, grouped):
    """Inputs of one read and its forward outputs (out, side, lse) from the
    library; with a token order, the side buffer when the read takes the pair
    path."""
    lib = _lib.load()
    g = torch.Generator().manual_seed(seed)
    L, D = E * BS, H * HD
    q = torch.randn(B, S, H, HD, generator=g).bfloat16().to(dev)
    k = torch.randn(L, D, generator=g).bfloat16().to(dev)
    v = torch.randn(L, D, generator=g).bfloat16().to(dev)
    idx = torch.rand(B, S, E, generator=g).argsort(-1)[..., :K].to(torch.int32).contiguous().to(dev)
    gates = torch.softmax(torch.randn(B, S, K, generator=g), -1).to(dev)
    dout = torch.randn(B, S, H, HD, generator=g).bfloat16().to(dev)
    order = None
    st = _lib.stream_of(dev)
    if grouped:
        order = torch.empty(int(lib.naylis_mom_read_order_words(B, S, E, K)), dtype=torch.int32, device=dev)
        ows = torch.empty(lib.naylis_mom_read_order_workspace_bytes(B, S, E, K), dtype=torch.uint8, device=dev)
        _lib.check(lib.naylis_mom_read_order(idx.data_ptr(), order.data_ptr(), ows.data_ptr(), ows.numel(), B, S, E,
                                             K, st))
    out = torch.empty_like(q)
    side_bytes = int(lib.naylis_mom_read_side_bytes(B, S, H, HD, E, BS, K))
    side = torch.empty(side_bytes, dtype=torch.uint8, device=dev) if grouped and side_bytes else None
    lse = torch.empty(H, B, S, dtype=torch.float32, device=dev)
    _lib.check(lib.naylis_mom_read_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), idx.data_ptr(), gates.data_ptr(),
                                       None if order is None else order.data_ptr(), out.data_ptr(),
                                       None if side is None else side.data_ptr(), lse.data_ptr(),
                                       None, 0, B, S, H, HD, E, BS, K, st))
    return dict(q=q, k=k, v=v, idx=idx, gates=gates, order=order, out=out, side=side, lse=lse, dout=dout,
                dims=(B, S, H, HD, E, BS, K))


def _outputs(c):
    """dq, dk, dv, dgates buffers pre-filled with NaN, so a word left unwritten shows."""
    nan = float("nan")
    return (torch.full_like(c["q"], nan), torch.full_like(c["k"], nan), torch.full_like(c["v"], nan),
            torch.full_like(c["gates"], nan))


def _args(c, outs):
    dq, dk, dv, dg = outs
    return (c["q"].data_ptr(), c["k"].data_ptr(), c["v"].data_ptr(), c["idx"].data_ptr(), c["gates"].data_ptr(),
            None if c["order"] is None else c["order"].data_ptr(), c["out"].data_ptr(),
            None if c["side"] is None else c["side"].data_ptr(), c["lse"].data_ptr(),
            c["dout"].data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), dg.data_ptr())


def test_read_bwd_noalloc_matches_workspace_entry_point(dev):
    lib = _lib.load()
    st = _lib.stream_of(dev)
    with _lib.on_device(dev):
        # the config-4 read (24 heads, 32 blocks, 16384 tokens, top-2, sequence order: the
        # two-pass backward), then a config-2-like read (16 heads of 64, 8 blocks of 128 slots,
        # grouped token order: the pair-tiled backward), then a smaller, ragged one (4 heads of
        # 32, 4 blocks of 64 slots, 300 tokens): each call needs less scratch than the one before
        cases = [_case(dev, 4, 4096, 24, 64, 32, 128, 2, seed=4, grouped=False),
                 _case(dev, 4, 2048, 16, 64, 8, 128, 2, seed=1, grouped=True),
                 _case(dev, 1, 300, 4, 32, 4, 64, 2, seed=2, grouped=False)]
        assert cases[0]["side"] is None and cases[1]["side"] is not None
        needs = [lib.naylis_mom_read_workspace_bytes(*c["dims"]) for c in cases]
        assert 0 < needs[2] < needs[1] < needs[0] <= _max_bytes(), needs
        got = []
        for c in cases:                               # the two no-allocation calls, in a row
            outs = _outputs(c)
            _lib.check(lib.naylis_mom_read_bwd_noalloc(*_args(c, outs), *c["dims"], st))
            got.append(outs)
        torch.cuda.synchronize(dev)
        for c, need, outs in zip(cases, needs, got):
            want = _outputs(c)
            ws = torch.empty(need, dtype=torch.uint8, device=dev)
            _lib.check(lib.naylis_mom_read_bwd(*_args(c, want), ws.data_ptr(), ws.numel(), *c["dims"], st))
            torch.cuda.synchronize(dev)
            for name, a, b in zip(("dq", "dk", "dv", "dgates"), outs, want):
                assert torch.isfinite(b).all(), name
                assert torch.equal(a, b), f"{name} of {c['dims']}: max |diff| {float((a.float() - b.float()).abs().max())}"


def test_read_bwd_noalloc_rejects_reads_beyond_its_scratch(dev):
    """A read whose workspace exceeds the scratch array is refused with
    NAYLIS_ERR_WORKSPACE before anything runs; the next call still works."""
    lib = _lib.load()
    dims = (1, 64, 16, 128, 128, 128, 2)              # 16384 slots of 16 x 128: ~320 MiB of dK/dV partials
    assert lib.naylis_mom_read_workspace_bytes(*dims) > _max_bytes()
    with _lib.on_device(dev):
        rc = lib.naylis_mom_read_bwd_noalloc(*([1] * 14), *dims, _lib.stream_of(dev))
    assert rc == _lib.NAYLIS_ERR_WORKSPACE
    assert b"scratch" in lib.naylis_mom_last_error()
    c = _case(dev, 1, 128, 2, 64, 4, 32, 2, seed=3, grouped=False)
    a, b = _outputs(c), _outputs(c)
    st = _lib.stream_of(dev)
    with _lib.on_device(dev):
        _lib.check(lib.naylis_mom_read_bwd_noalloc(*_args(c, a), *c["dims"], st))
        ws = torch.empty(lib.naylis_mom_read_workspace_bytes(*c["dims"]), dtype=torch.uint8, device=dev)
        _lib.check(lib.naylis_mom_read_bwd(*_args(c, b), ws.data_ptr(), ws.numel(), *c["dims"], st))
    torch.cuda.synchronize(dev)
    assert all(torch.equal(x, y) for x, y in zip(a, b))
