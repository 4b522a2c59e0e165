"""Host-side checks that need no GPU: the C-ABI library loads and exports every symbol
include/moe_mi355x.h declares, argument validation, workspace and tile-count formulas."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

from oracle import moe_oracle as orc

ROOT = Path(__file__).resolve().parents[1]


def _declared_symbols():
    text = (ROOT / "include" / "moe_mi355x.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(moe_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_entry_points():
    names = _declared_symbols()
    assert "moe_block_forward" in names and "moe_route_topk" in names and len(names) >= 14


def test_library_exports_every_declared_symbol(pkg):
    lib = pkg._lib.load()
    for name in _declared_symbols():
        assert hasattr(lib, name), name
        assert name in pkg._lib.SIGNATURES, f"{name} has no ctypes signature"
    assert set(pkg._lib.SIGNATURES) == set(_declared_symbols())
    assert lib.moe_abi_version() == pkg._lib.ABI_VERSION == 3


@pytest.mark.parametrize("T,k,E,bm,sh", [(1, 8, 256, 64, 1), (64, 8, 256, 64, 1),
                                          (4096, 8, 256, 64, 0), (0, 4, 16, 64, 1), (3, 2, 4, 2, 1)])
def test_max_tiles_formula(pkg, T, k, E, bm, sh):
    assert pkg._lib.load().moe_max_tiles(T, k, E, bm, sh) == orc.max_tiles(T, k, E, bm, bool(sh))


def test_workspace_grows_with_tokens(pkg):
    lib = pkg._lib.load()
    a = lib.moe_block_workspace_bytes(1, 2048, 256, 8, 512, 512, 272)
    b = lib.moe_block_workspace_bytes(64, 2048, 256, 8, 512, 512, 272)
    assert 0 < a < b
    # the pair outputs [P, H] and activations [P, I] dominate
    assert b >= 64 * 8 * (2048 + 512) * 2
    assert lib.moe_experts_workspace_bytes(16, 128, 16, 4, 64) > 0


def test_invalid_arguments_raise_before_any_launch(pkg):
    lib = pkg._lib.load()
    rc = lib.moe_route_topk(None, 16, 4, 16, 99, None, None, None, None)
    assert rc == pkg._lib.MOE_EINVAL
    assert b"top_k" in lib.moe_last_error()
    rc = lib.moe_experts_forward(None, 4, 100, 16, 4, 64, None, None, None, None, None, None, 0, 1,
                                 None, None, 0, None)
    assert rc == pkg._lib.MOE_EINVAL and b"hidden" in lib.moe_last_error()
    rc = lib.moe_combine(None, None, 1, 2048, 8, None, None, 0, None, None, 7, None)
    assert rc == pkg._lib.MOE_EINVAL


def test_cpu_tensors_fail_loudly(pkg):
    x = torch.zeros(2, 64, dtype=torch.bfloat16)
    with pytest.raises(pkg.MoeLibraryError, match="no CPU path"):
        pkg.ops.route(x, 2)


def test_supported_predicate(pkg):
    x = torch.zeros(2, 64, dtype=torch.bfloat16)
    gu = torch.zeros(4, 64, 64, dtype=torch.bfloat16)
    dn = torch.zeros(4, 64, 32, dtype=torch.bfloat16)
    assert not pkg.ops.supported(x, gu, dn)  # CPU tensor


def test_fp8_quantize_matches_oracle(pkg):
    g = torch.Generator().manual_seed(0)
    w = (torch.randn(3, 32, 64, generator=g) * 0.02).to(torch.bfloat16)
    q, s = pkg.fp8.quantize_rows(w)
    q2, s2 = orc.quantize_rows(w)
    assert torch.equal(q.view(torch.uint8), q2.view(torch.uint8)) and torch.equal(s, s2)
    assert q.dtype == torch.float8_e4m3fn and s.shape == (3, 32)


def test_decode_fits_predicate(pkg):
    """The decode path's shape limits: T <= 4, T*k <= 64, H a multiple of 512 up to 4096,
    I and IS in {512, 1024}, E <= 512 (routing inside the launch)."""
    fits = pkg.ops.decode_fits
    assert fits(1, 2048, 256, 8, 512, 512)
    assert fits(4, 2048, 256, 8, 512, 512)
    assert fits(4, 4096, 512, 16, 1024, 1024)
    assert not fits(5, 2048, 256, 8, 512, 512)
    assert not fits(0, 2048, 256, 8, 512, 512)
    assert not fits(1, 2048 + 256, 256, 8, 512, 512)
    assert not fits(1, 8192, 256, 8, 512, 512)
    assert not fits(1, 2048, 256, 8, 256, 512)
    assert not fits(1, 2048, 256, 8, 512, 768)
    assert not fits(1, 2048, 1024, 8, 512, 512)
    assert not fits(4, 2048, 256, 17, 512, 512)


def test_add_rms_argument_checks_before_any_launch(pkg):
    """moe_add_rmsnorm / moe_block_forward_add_rms reject bad shapes, missing buffers,
    aliasing and misalignment with MOE_EINVAL before touching the device (the addresses
    here are never dereferenced)."""
    lib = pkg._lib.load()
    EINVAL = pkg._lib.MOE_EINVAL
    X, Hh, W, TOT, OUT = 0x10000, 0x20000, 0x30000, 0x40000, 0x50000
    T, H = 2, 64
    assert lib.moe_add_rmsnorm(X, None, W, T, 60, 1e-6, None, OUT, None) == EINVAL  # H % 8
    assert lib.moe_add_rmsnorm(X, None, W, T, 8192 + 8, 1e-6, None, OUT, None) == EINVAL
    assert lib.moe_add_rmsnorm(X, Hh, W, T, H, 1e-6, None, OUT, None) == EINVAL  # no total
    assert lib.moe_add_rmsnorm(X, None, W, T, H, -1.0, None, OUT, None) == EINVAL  # eps
    assert lib.moe_add_rmsnorm(X, None, W, T, H, 1e-6, None, X + 64, None) == EINVAL  # overlap
    assert lib.moe_add_rmsnorm(X, Hh, W, T, H, 1e-6, OUT, OUT + 2, None) == EINVAL  # overlap
    assert lib.moe_add_rmsnorm(X + 2, None, W, T, H, 1e-6, None, OUT, None) == EINVAL  # align
    assert b"add_rms" in lib.moe_last_error()
    P = 0x60000
    ws = 1 << 20
    args = (T, 2048, 256, 8, 512, 512, P, 272, P, None, P, None, 0, P, P + 2048 * 512 * 2, P,
            1)
    # norm output overlapping the block output
    assert lib.moe_block_forward_add_rms(X, Hh, W, 1e-6, *args, TOT, OUT, OUT, None, None,
                                         None, P, ws, None) == EINVAL
    # total overlapping the input
    assert lib.moe_block_forward_add_rms(X, Hh, W, 1e-6, *args, X, OUT, OUT + (1 << 16), None,
                                         None, None, P, ws, None) == EINVAL


@pytest.mark.parametrize("H,fits", [(512, 1), (1024, 1), (2048, 1), (4096, 1), (1536, 0),
                                    (2560, 0), (3072, 0), (3584, 0), (8192, 0)])
def test_decode_fits_only_instantiated_hidden_sizes(pkg, H, fits):
    """The decode kernels are instantiated for H = 512 x {1, 2, 4, 8}; other multiples of
    512 go to the tiled path instead of failing at launch."""
    assert pkg._lib.load().moe_decode_fits(1, H, 256, 8, 512, 512) == fits


def test_noalloc_rejects_calls_beyond_its_scratch_before_any_launch(pkg):
    """moe_block_forward_noalloc checks the call's workspace against the static scratch
    (MOE_NOALLOC_SCRATCH_BYTES) before touching the GPU: too many tokens fail with MOE_EINVAL
    and a message naming the limit; the header's size and the Python constant agree."""
    lib = pkg._lib.load()
    hdr = (ROOT / "include" / "moe_mi355x.h").read_text()
    assert re.search(r"#define MOE_NOALLOC_SCRATCH_BYTES \(16u << 20\)", hdr)
    H, E, K, I, NP = 2048, 256, 8, 512, 320
    T = 1
    while lib.moe_block_workspace_bytes(T, H, E, K, I, I, NP) <= pkg._lib.NOALLOC_SCRATCH_BYTES:
        T *= 2
    rc = lib.moe_block_forward_noalloc(None, T, H, E, K, I, I, None, NP, None, None, None, None,
                                       0, None, None, None, None, 0, None, None, None, None, None)
    assert rc == pkg._lib.MOE_EINVAL
    assert b"static scratch" in lib.moe_last_error()
    rc = lib.moe_block_forward_noalloc(None, -1, H, E, K, I, I, None, NP, None, None, None, None,
                                       0, None, None, None, None, 0, None, None, None, None, None)
    assert rc == pkg._lib.MOE_EINVAL


def test_probe_library_loads():
    """bench.py's read-ceiling probe is built beside the MoE library and exports its entry;
    it rejects bad arguments on the host (no GPU call)."""
    import ctypes
    from pathlib import Path

    path = Path(__file__).resolve().parent.parent / "qwen36-mi250-tracelab-20261107_amd" / "libmoe_probe.so"
    if not path.exists():
        pytest.skip("libmoe_probe.so not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(str(path))
    fn = lib.moe_probe_stream_read
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p, ctypes.c_longlong, ctypes.c_void_p, ctypes.c_int,
                   ctypes.c_void_p]
    assert fn(None, 16, None, 1, None) == 1
    assert fn(ctypes.c_void_p(16), 15, ctypes.c_void_p(16), 1, None) == 1
