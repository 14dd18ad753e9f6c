"""CPU checks of the C-ABI library (no GPU calls): it loads, exports every
function include/naylis_mom.h declares, and rejects bad arguments with the
reference's fail-loud rules (mom_kernels/triton_gpu.py:420-429,
mom_kernels/__init__.py:69-79) as status codes — before touching a device.
Also the Python-side contracts of resolve_mode / preflight / mom_read
(tests/test_parity.py §7-8) and the layer constructor (model.py:125-133).
"""
import ctypes
import os
import re

import pytest
import torch

from naylis_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "naylis_mom.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(naylis_mom_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_library_exports_every_declared_symbol(lib):
    names = declared_functions()
    assert len(names) >= 12
    raw = ctypes.CDLL(_lib.LIB_PATH)
    for n in names:
        assert hasattr(raw, n), f"{n} declared in include/naylis_mom.h but not exported"
    assert set(names) == set(_lib.SIGNATURES), "ctypes signature table out of sync with the header"


def test_torch_extension_loads(lib):
    """The fused layer node's torch extension (csrc/torch_layer.cpp) loads
    against the library and exports its two calls (no device work)."""
    from naylis_amd import _torch_ext
    ext = _torch_ext.load()
    assert callable(ext.layer_fwd) and callable(ext.layer_bwd)


def test_abi_version(lib):
    assert lib.naylis_mom_abi_version() == _lib.ABI_VERSION


def test_spin_limit_setter(lib):
    """The one-launch router's poll bound: a negative argument reads it, any
    other sets it and returns the previous bound (host state only)."""
    cur = lib.naylis_mom_spin_limit(-1)
    assert cur == 20000
    assert lib.naylis_mom_spin_limit(0) == cur
    assert lib.naylis_mom_spin_limit(-5) == 0
    assert lib.naylis_mom_spin_limit(cur) == 0
    assert lib.naylis_mom_spin_limit(-1) == cur


READ_OK = dict(B=2, S=64, H=2, hd=16, nb=4, bs=16, k=2)


def read_fwd(lib, **kw):
    a = dict(READ_OK, **kw)
    return lib.naylis_mom_read_fwd(1, 1, 1, 1, 1, None, 1, None, 1, None, 0, a["B"], a["S"], a["H"], a["hd"],
                                   a["nb"], a["bs"], a["k"], None)


@pytest.mark.parametrize("bad", [dict(hd=96), dict(hd=256), dict(hd=8), dict(k=0), dict(k=9), dict(k=5, nb=4),
                                 dict(nb=0), dict(bs=0), dict(nb=2048), dict(B=-1), dict(H=0)])
def test_read_rejects_bad_arguments(lib, bad):
    rc = read_fwd(lib, **bad)
    assert rc == _lib.NAYLIS_ERR_ARG
    assert lib.naylis_mom_last_error()
    assert lib.naylis_mom_read_workspace_bytes(*[dict(READ_OK, **bad)[n] for n in ("B", "S", "H", "hd", "nb", "bs",
                                                                                     "k")]) == 0


def test_read_null_pointers_and_workspace(lib):
    rc = lib.naylis_mom_read_fwd(None, None, None, None, None, None, None, None, None, None, 0, 2, 64, 2, 16, 4, 16,
                                 2, None)
    assert rc == _lib.NAYLIS_ERR_ARG and b"null" in lib.naylis_mom_last_error()
    # both backward paths refuse a workspace one byte short of the query: the two-pass kernels
    # (16 blocks) and the pair-tiled ones (8 blocks, an order and a side buffer given)
    for nb in (16, 8):
        ws = lib.naylis_mom_read_workspace_bytes(8, 2048, 16, 64, nb, 128, 2)
        assert ws > 0
        rc = lib.naylis_mom_read_bwd(*([1] * 14), 1, ws - 1, 8, 2048, 16, 64, nb, 128, 2, None)
        assert rc == _lib.NAYLIS_ERR_WORKSPACE, nb
    # empty sequences are a valid no-op for the forward
    assert lib.naylis_mom_read_fwd(None, None, None, None, None, None, None, None, None, None, 0, 2, 0, 2, 16, 4, 16,
                                   2, None) == _lib.NAYLIS_OK
    # the token order: argument checks, workspace, empty input
    assert lib.naylis_mom_read_order_workspace_bytes(8, 2048, 8, 2) > 0
    assert lib.naylis_mom_read_order_workspace_bytes(8, 2048, 8, 9) == 0
    assert lib.naylis_mom_read_order(1, 1, 1, 1, 8, 2048, 8, 2, None) == _lib.NAYLIS_ERR_WORKSPACE
    assert lib.naylis_mom_read_order(None, None, None, 0, 0, 2048, 8, 2, None) == _lib.NAYLIS_OK
    # the order buffer: 1 + N words, plus the pair plan for top-2 over at most 32 blocks
    N = 8 * 2048
    assert lib.naylis_mom_read_order_words(8, 2048, 8, 3) == 1 + N
    assert lib.naylis_mom_read_order_words(8, 2048, 64, 2) == 1 + N
    plan = lib.naylis_mom_read_order_words(8, 2048, 8, 2)
    keys = 8 * 9 // 2
    tiles = N // 32 + keys
    assert plan == ((1 + N + 3) // 4) * 4 + 8 + 4 * keys + 4 * tiles
    assert lib.naylis_mom_read_order_words(8, 2048, 8, 9) == 0


@pytest.mark.parametrize("dims,want", [
    ((8, 2048, 16, 64, 8, 128, 2), 1),    # config 2: the pair-tiled backward
    ((1, 300, 4, 64, 4, 128, 2), 1),      # ragged, 4 blocks
    ((4, 4096, 24, 64, 32, 128, 2), 0),   # config 4: 32 blocks (pair forward only)
    ((8, 2048, 16, 32, 8, 128, 2), 0),    # head_dim 32
    ((8, 2048, 16, 64, 8, 64, 2), 0),     # 64-slot blocks
    ((8, 2048, 16, 64, 8, 128, 3), 0),    # top-3
    ((8, 0, 16, 64, 8, 128, 2), 0),       # no tokens
])
def test_read_side_bytes_rule(lib, dims, want):
    """naylis_mom_read_side_bytes > 0 exactly where the pair-tiled backward
    applies: four 32-bit row constants per (head, token)."""
    nbytes = lib.naylis_mom_read_side_bytes(*dims)
    assert (nbytes > 0) == bool(want)
    if want:
        B, S, H = dims[:3]
        assert nbytes == B * S * H * 16


def test_router_and_bank_reject_bad_arguments(lib):
    assert lib.naylis_mom_router_workspace_bytes(2, 64, 32, 65, 8, 2) == 0     # rank > 64
    assert lib.naylis_mom_router_workspace_bytes(2, 64, 32, 8, 65, 2) == 0     # blocks > 64
    assert lib.naylis_mom_router_workspace_bytes(2, 64, 32, 8, 4, 5) == 0      # top_k > blocks
    assert lib.naylis_mom_router_workspace_bytes(2, 64, 32, 8, 4, 2) > 0
    rc = lib.naylis_mom_router_fwd(1, 7, 1, 1, None, 0, 1.0, 1, 1, 1, 1, 1, None, 1, 1 << 30, 2, 64, 32, 8, 4, 2,
                                   None)
    assert rc == _lib.NAYLIS_ERR_ARG                                           # unknown dtype code
    rc = lib.naylis_mom_router_fwd(1, 1, 1, 1, 1, 2, 1.0, 1, 1, 1, 1, 1, None, 1, 1 << 30, 2, 64, 32, 8, 4, 2,
                                   None)
    assert rc == _lib.NAYLIS_ERR_ARG                                           # unknown noise kind
    rc = lib.naylis_mom_router_bwd(1, 1, 1, 1, 1, 1, 1, 1, None, 1, 3, None, 1, 0, 1, 1, 1, 1 << 30, 2, 64, 32, 8,
                                   4, 2, None)
    assert rc == _lib.NAYLIS_ERR_ARG                                           # d_probs stride not E or 0
    assert lib.naylis_mom_router_stats_workspace_bytes(100, 8) > 0
    assert lib.naylis_mom_router_stats_workspace_bytes(100, 65) == 0
    assert lib.naylis_mom_router_stats(1, 1, 1, 1, 1 << 20, 100, 8, 9, None) == _lib.NAYLIS_ERR_ARG  # top_k > E
    assert lib.naylis_mom_router_stats(1, 1, 1, 1, 0, 100, 8, 2, None) == _lib.NAYLIS_ERR_WORKSPACE
    assert lib.naylis_mom_router_stats(None, None, 1, None, 0, 0, 8, 2, None) == _lib.NAYLIS_ERR_ARG  # no workspace


def test_rmsnorm_rejects_bad_arguments(lib):
    p = 0x1000
    assert lib.naylis_mom_rmsnorm_workspace_bytes(16384, 1024) > 0
    assert lib.naylis_mom_rmsnorm_workspace_bytes(16384, 1000) == 0
    assert lib.naylis_mom_rmsnorm_fwd(p, 1, p, p, p, 8, 1000, 1e-5, None) == _lib.NAYLIS_ERR_ARG    # D % 512
    assert lib.naylis_mom_rmsnorm_fwd(p, 1, p, p, p, 8, 8192, 1e-5, None) == _lib.NAYLIS_ERR_ARG    # D > 4096
    assert lib.naylis_mom_rmsnorm_fwd(p, 3, p, p, p, 8, 1024, 1e-5, None) == _lib.NAYLIS_ERR_ARG    # dtype
    assert lib.naylis_mom_rmsnorm_fwd(p, 1, p, p, p, 8, 1024, -1.0, None) == _lib.NAYLIS_ERR_ARG    # eps
    assert lib.naylis_mom_rmsnorm_fwd(p + 2, 1, p, p, p, 8, 1024, 1e-5, None) == _lib.NAYLIS_ERR_ARG  # alignment
    assert lib.naylis_mom_rmsnorm_fwd(None, 1, None, None, None, 0, 1024, 1e-5, None) == _lib.NAYLIS_OK
    assert lib.naylis_mom_rmsnorm_bwd(p, 1, p, p, p, p, p, p, 0, 8, 1024, None) == _lib.NAYLIS_ERR_WORKSPACE
    assert lib.naylis_mom_bank_kv_fwd(1, 1, 1, 1, 1, 64, 30, 32, None) == _lib.NAYLIS_ERR_ARG   # D_in % 8
    assert lib.naylis_mom_bank_kv_fwd(None, None, None, None, None, 0, 32, 32, None) == _lib.NAYLIS_OK
    assert lib.naylis_mom_bank_kv_bwd(1, 1, 1, 1, 1, 1, 9, 1, 1, 0, 64, 32, 32, None) == _lib.NAYLIS_ERR_ARG


DEC_OK = dict(B=64, D=1024, H=16, R=32, E=8, bs=128, k=2)


def decode(lib, state_out=0x2000000, x_dtype=1, **kw):
    a = dict(DEC_OK, **kw)
    p = 0x1000  # 16-byte aligned stand-in pointers: validation runs before any device work
    return lib.naylis_mom_decode_step(0x1000000, state_out, p, p, x_dtype, p, p, p, p, p, p, p, p, p, p, a["B"],
                                      a["D"], a["H"], a["R"], a["E"], a["bs"], a["k"], None)


@pytest.mark.parametrize("bad", [dict(H=12), dict(D=1000), dict(H=64), dict(D=8192, H=64), dict(R=65),
                                 dict(R=0), dict(E=65), dict(k=0), dict(k=9), dict(k=3, E=2), dict(bs=0),
                                 dict(bs=4096), dict(B=-1), dict(x_dtype=5), dict(state_out=0x1000400)])
def test_decode_rejects_bad_arguments(lib, bad):
    assert decode(lib, **bad) == _lib.NAYLIS_ERR_ARG
    assert lib.naylis_mom_last_error().startswith(b"decode_step")
    assert decode(lib, B=0) == _lib.NAYLIS_OK  # nothing to do, no pointer touched


def test_bank_quant_rejects_bad_arguments(lib):
    assert lib.naylis_mom_bank_quant_fp8(1, 1, 1, 1, 1, 1, -1, 64, None) == _lib.NAYLIS_ERR_ARG
    assert lib.naylis_mom_bank_quant_fp8(1, 1, 1, 1, 1, 1, 64, 0, None) == _lib.NAYLIS_ERR_ARG
    assert lib.naylis_mom_bank_quant_fp8(None, 1, 1, 1, 1, 1, 64, 64, None) == _lib.NAYLIS_ERR_ARG
    assert lib.naylis_mom_bank_quant_fp8(None, None, None, None, None, None, 0, 64, None) == _lib.NAYLIS_OK


def test_error_message_is_per_thread(lib):
    import threading
    read_fwd(lib, hd=96)
    msgs = {}

    def other():
        read_fwd(lib, k=0)
        msgs["t"] = lib.naylis_mom_last_error()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert b"head_dim" in lib.naylis_mom_last_error()
    assert b"top_k" in msgs["t"]


# ------------------------------------------------------- python contracts
def test_resolve_mode_contract():
    from naylis_amd import mom_kernels
    with pytest.raises(RuntimeError):
        mom_kernels.resolve_mode(torch.device("cpu"), torch.float32)               # §7a
    with pytest.raises(RuntimeError):
        mom_kernels.resolve_mode("cuda", torch.float32, head_dim=64)               # §7b
    with pytest.raises(RuntimeError):
        mom_kernels.resolve_mode("cuda", torch.bfloat16, head_dim=96)              # §7c
    with pytest.raises(RuntimeError):
        mom_kernels.resolve_mode("xla", torch.float32, head_dim=64)                # no XLA backend here
    if torch.version.hip is not None and _lib.available():
        assert mom_kernels.resolve_mode("cuda", torch.bfloat16, head_dim=64) == "hip"   # §7d
    with pytest.raises(RuntimeError):
        mom_kernels.preflight("cpu")                                             # §8a
    with pytest.raises(RuntimeError):
        mom_kernels.mom_read(None, None, None, None, None, num_blocks=1, block_size=1, mode="triton")


def test_mom_read_preconditions_raise_before_device_work():
    from naylis_amd import mom_kernels
    q = torch.zeros(2, 8, 2, 16, dtype=torch.bfloat16)
    k = torch.zeros(64, 32, dtype=torch.bfloat16)
    top = torch.zeros(2, 8, 2, dtype=torch.long)
    g = torch.full((2, 8, 2), 0.5)
    with pytest.raises(RuntimeError, match="shared K/V"):
        mom_kernels.mom_read(q, k.unsqueeze(0), k, top, g, num_blocks=4, block_size=16, mode="hip")
    with pytest.raises(RuntimeError, match="bf16"):
        mom_kernels.mom_read(q.float(), k, k, top, g, num_blocks=4, block_size=16, mode="hip")
    with pytest.raises(RuntimeError, match="slots"):
        mom_kernels.mom_read(q, k, k, top, g, num_blocks=3, block_size=16, mode="hip")
    with pytest.raises(RuntimeError, match="ROCm device"):
        mom_kernels.mom_read(q, k, k, top, g, num_blocks=4, block_size=16, mode="hip")


def test_layer_constructor_contract():
    from naylis_amd.layer import MoMLayer
    with pytest.raises(ValueError):
        MoMLayer(d_model=30, n_heads=4, mem_size=64, block_size=16, top_blocks=2, router_rank=8)
    with pytest.raises(ValueError):
        MoMLayer(d_model=32, n_heads=2, mem_size=60, block_size=16, top_blocks=2, router_rank=8)
    with pytest.raises(ValueError):
        MoMLayer(d_model=32, n_heads=2, mem_size=64, block_size=16, top_blocks=5, router_rank=8)
    layer = MoMLayer(d_model=32, n_heads=2, mem_size=64, block_size=16, top_blocks=2, router_rank=8)
    names = {n for n, _ in layer.named_parameters()}
    assert names == {"router_down.weight", "router_up.weight", "q_proj.weight", "k_proj.weight", "v_proj.weight",
                     "o_proj.weight", "mom_scale"}                               # checkpoint-compatible names
    with pytest.raises(RuntimeError):
        layer(torch.zeros(1, 4, 32), torch.zeros(4, 16 * 32))                   # CPU tensors: no fallback


def test_rope_rejects_bad_arguments(lib):
    p = 0x1000
    assert lib.naylis_mom_rope(p, p, p, p, p, p, 1, 0, 2, 8, 4, 48, 1, None) == _lib.NAYLIS_ERR_ARG   # head_dim
    assert lib.naylis_mom_rope(p, p, p, p, p, p, 1, 0, 2, 8, 4, 64, 3, None) == _lib.NAYLIS_ERR_ARG   # cos batch
    assert lib.naylis_mom_rope(p, p, p, p, p, p, 5, 0, 2, 8, 4, 64, 1, None) == _lib.NAYLIS_ERR_ARG   # dtype
    assert lib.naylis_mom_rope(None, p, p, p, p, p, 1, 0, 2, 8, 4, 64, 1, None) == _lib.NAYLIS_ERR_ARG
    assert lib.naylis_mom_rope(None, None, None, None, None, None, 1, 0, 0, 8, 4, 64, 1, None) == _lib.NAYLIS_OK
    q, k, c, o = 0x100000, 0x200000, 0x300000, 0x400000
    assert lib.naylis_mom_rope(q, k, c, c, q, o, 1, 0, 2, 8, 4, 64, 1, None) == _lib.NAYLIS_ERR_ARG   # in place


def test_swiglu_rejects_bad_arguments(lib):
    p = 0x1000
    assert lib.naylis_mom_swiglu_fwd(p, p, p, 1, 12, None) == _lib.NAYLIS_ERR_ARG          # n % 8
    assert lib.naylis_mom_swiglu_fwd(p, p, p, 4, 16, None) == _lib.NAYLIS_ERR_ARG          # dtype
    assert lib.naylis_mom_swiglu_fwd(p + 4, p, p, 1, 16, None) == _lib.NAYLIS_ERR_ARG      # alignment
    assert lib.naylis_mom_swiglu_bwd(p, p, None, p, p, 1, 16, None) == _lib.NAYLIS_ERR_ARG
    assert lib.naylis_mom_swiglu_fwd(None, None, None, 1, 0, None) == _lib.NAYLIS_OK


def test_xent_rejects_bad_arguments(lib):
    p = 0x1000
    assert lib.naylis_mom_xent_fwd(p, p, p, p, 8, 1000, -100, None) == _lib.NAYLIS_ERR_ARG          # V % 2048
    assert lib.naylis_mom_xent_fwd(p + 2, p, p, p, 8, 2048, -100, None) == _lib.NAYLIS_ERR_ARG      # alignment
    assert lib.naylis_mom_xent_bwd(p, p, p, p, 2, p, 8, 2048, -100, None) == _lib.NAYLIS_ERR_ARG     # grad stride
    assert lib.naylis_mom_xent_fwd(None, None, None, None, 0, 2048, -100, None) == _lib.NAYLIS_OK


def test_add_rmsnorm_rejects_bad_arguments(lib):
    p = 0x1000
    # fp32 stream with a bf16 residual branch
    assert lib.naylis_mom_add_rmsnorm_fwd(p, p, 1, p, p, p, p, 0, 8, 1024, 1e-5, None) == _lib.NAYLIS_ERR_ARG
    assert lib.naylis_mom_add_rmsnorm_fwd(p, p, 0, p, p, p, p, 1, 8, 1000, 1e-5, None) == _lib.NAYLIS_ERR_ARG  # D
    assert lib.naylis_mom_add_rmsnorm_bwd(p, p, p, p, None, p, p, p, 0, 1, 8, 1024, None) == _lib.NAYLIS_ERR_WORKSPACE


def test_read_bwd_noalloc_refuses_before_touching_a_device(lib):
    """The no-allocation read backward checks shapes and its scratch limit
    (NAYLIS_READ_BWD_NOALLOC_MAX_BYTES) before any device call."""
    m = re.search(r"#define NAYLIS_READ_BWD_NOALLOC_MAX_BYTES \(\(size_t\)(\d+) << (\d+)\)", open(HEADER).read())
    max_bytes = int(m.group(1)) << int(m.group(2))
    dims = (1, 64, 16, 128, 128, 128, 2)              # 16384 slots of 16 x 128: 256 MiB of dK/dV partials
    assert lib.naylis_mom_read_workspace_bytes(*dims) > max_bytes
    assert lib.naylis_mom_read_bwd_noalloc(*([1] * 14), *dims, None) == _lib.NAYLIS_ERR_WORKSPACE
    assert b"scratch" in lib.naylis_mom_last_error()
    assert lib.naylis_mom_read_bwd_noalloc(*([1] * 14), 1, 64, 2, 96, 4, 16, 2, None) == _lib.NAYLIS_ERR_ARG


def test_bank_grouped_rejects_bad_arguments(lib):
    """The grouped bank projection refuses, before touching a device, layer
    counts outside [1, NAYLIS_BANK_GROUP_MAX_LAYERS], D_out not a multiple of
    64, null pointer arrays or entries, and a short workspace."""
    P = ctypes.c_void_p
    one = (P * 2)(1, 1)
    fwd = lib.naylis_mom_bank_kv_fwd_grouped
    assert fwd(1, one, one, one, one, 0, 64, 64, 64, None) == _lib.NAYLIS_ERR_ARG
    assert fwd(1, one, one, one, one, 25, 64, 64, 64, None) == _lib.NAYLIS_ERR_ARG
    assert fwd(1, one, one, one, one, 2, 64, 64, 96, None) == _lib.NAYLIS_ERR_ARG
    assert "D_out" in lib.naylis_mom_last_error().decode()
    assert fwd(1, None, one, one, one, 2, 64, 64, 64, None) == _lib.NAYLIS_ERR_ARG
    assert fwd(1, (P * 2)(1, None), one, one, one, 2, 64, 64, 64, None) == _lib.NAYLIS_ERR_ARG
    assert lib.naylis_mom_bank_kv_bwd_grouped_workspace_bytes(2, 64, 32, 64) == 2 * 64 * 32 * 4
    assert lib.naylis_mom_bank_kv_bwd_grouped_workspace_bytes(0, 64, 32, 64) == 0
    bwd = lib.naylis_mom_bank_kv_bwd_grouped
    f32, bf16 = 0, 1  # NAYLIS_DTYPE_F32, NAYLIS_DTYPE_BF16
    args = [1, one, one, one, one, 1, f32, one, one, bf16]
    assert bwd(*args, None, 0, 2, 64, 32, 64, None) == _lib.NAYLIS_ERR_WORKSPACE
    assert bwd(*args, 1, 2 * 64 * 32 * 4 - 1, 2, 64, 32, 64, None) == _lib.NAYLIS_ERR_WORKSPACE
    assert bwd(*args, 1, 1 << 20, 25, 64, 32, 64, None) == _lib.NAYLIS_ERR_ARG
