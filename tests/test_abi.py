"""CPU checks of the C ABI: libqlka.so builds for gfx950, loads, exports every function include/qlka.h declares, and
its host-side validation answers without touching a GPU (no compute call is made here)."""

import ctypes
import os
import re

import pytest

from qlka import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "qlka.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(qlka_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        from qlka import build
        build.build()
    return _lib.load()


def test_header_declares_the_boundary():
    names = _declared()
    for fn in ("qlka_laplace_fwd", "qlka_abs_fwd", "qlka_abs_bwd", "qlka_sgn_fwd", "qlka_seg_sort",
               "qlka_merge_rank", "qlka_last_error"):
        assert fn in names


def test_every_declared_symbol_is_exported(lib):
    raw = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in _declared() if not hasattr(raw, n)]
    assert not missing, f"not exported: {missing}"
    assert set(_declared()) == set(_lib.EXPORTED), "ctypes signature table out of sync with include/qlka.h"


def test_version_and_workspace_sizes(lib):
    assert lib.qlka_version() == 1
    small = lib.qlka_laplace_fwd_ws_bytes(1, 1, 800, 800, 4)
    big = lib.qlka_laplace_fwd_ws_bytes(12, 64, 16384, 16384, 64)
    assert 0 < small < big
    # calls the dense route takes (at the default cutoff 512) need no workspace
    assert lib.qlka_laplace_fwd_ws_bytes(1, 1, 8, 8, 4) == 0
    assert lib.qlka_abs_bwd_ws_bytes(32, 64, 600, 600, 64) == 0
    assert lib.qlka_sgn_fwd_ws_bytes(2, 3, 500, 500, 8) == 0
    assert lib.qlka_abs_fwd_ws_bytes(32, 64, 1024, 1024, 64) == 0        # dense below 2 x the cutoff
    assert lib.qlka_abs_fwd_ws_bytes(65535, 64, 512, 512, 64) == 0
    assert lib.qlka_abs_fwd_ws_bytes(2, 3, 9, 100000, 8) == 0            # 16 keys or fewer: dense at any length
    assert lib.qlka_abs_bwd_ws_bytes(12, 64, 600, 600, 64) > 0          # too few workgroups at L = 600: walks
    prev = lib.qlka_set_direct_max(0)
    try:
        assert lib.qlka_laplace_fwd_ws_bytes(1, 1, 8, 8, 4) > 0          # cutoff 0: always sort and walk
        assert lib.qlka_abs_fwd_ws_bytes(1, 1, 17, 8, 4) > 0
        # ... except segments of at most 16 keys, which the abs sums always take dense
        assert lib.qlka_abs_fwd_ws_bytes(1, 1, 16, 8, 4) == 0
        assert lib.qlka_abs_bwd_ws_bytes(1, 1, 16, 800, 4) == 0
        assert lib.qlka_abs_bwd_walks(1, 800, 16) == 0
    finally:
        lib.qlka_set_direct_max(prev)
    # the row-emitting ops carry one contribution row per (p, d, query) of a chunk: the D-fold slab
    assert lib.qlka_laplace_fwd_ws_bytes(1, 64, 16384, 16384, 64) >= 64 * 16384 * 64 * 4
    assert lib.qlka_abs_bwd_ws_bytes(1, 64, 16384, 16384, 64) >= 64 * 16384 * 64 * 4
    assert lib.qlka_sgn_fwd_ws_bytes(1, 64, 16384, 16384, 64) < 64 * 16384 * 64 * 4
    # the global (multi-run) sort needs scratch, the LDS sort none
    assert lib.qlka_seg_sort_ws_bytes(4, 16384) == 0
    assert lib.qlka_seg_sort_ws_bytes(4, 16385) > 0
    assert lib.qlka_laplace_fwd_ws_bytes(0, 1, 1, 1, 1) == 0


def test_workspace_budget_sizes_the_queries(lib):
    """The budget picks the chunking of a call; no GPU is touched. At the headline shape a call is pipelined: three
    chunks of four p with two workspace copies; below that budget, smaller chunks with two copies, and one p with one
    copy when two do not fit."""
    prev = lib.qlka_set_workspace_budget(8 << 30)
    try:
        dims = (12, 64, 16384, 16384, 64)
        one = lib.qlka_laplace_fwd_ws_bytes(1, *dims[1:])       # one p: not pipelined, one copy
        full = lib.qlka_laplace_fwd_ws_bytes(*dims)
        assert abs(full - 2 * 4 * one) < 64 << 10                 # two copies of a 4-p chunk (alignment slack)
        assert lib.qlka_set_workspace_budget(1) == 8 << 30
        assert lib.qlka_laplace_fwd_ws_bytes(*dims) == one
        assert lib.qlka_abs_bwd_ws_bytes(*dims) == lib.qlka_abs_bwd_ws_bytes(1, *dims[1:])
        lib.qlka_set_workspace_budget(3 * one + 10)
        assert lib.qlka_laplace_fwd_ws_bytes(*dims) == 2 * one   # two copies of a 1-p chunk
        lib.qlka_set_workspace_budget(1 << 62)
        assert lib.qlka_laplace_fwd_ws_bytes(*dims) == full
    finally:
        lib.qlka_set_workspace_budget(prev)


def test_config4_backward_pipelines_under_the_default_budget(lib):
    """At configs[4] (N = M = 131072, C = 64) one p's merged-backward workspace fits twice in the 5 GiB default budget
    (its own sorts share the slab region), so the backward runs two copies of one-p chunks, each chunk's grad_v reduce
    beside the next chunk's work; the forwards too."""
    prev = lib.qlka_set_workspace_budget(5 << 30)
    try:
        dims = (12, 64, 131072, 131072, 64)
        one = lib.qlka_abs_bwd_ws_bytes(1, *dims[1:])              # one p: not pipelined, one copy
        assert lib.qlka_abs_bwd_ws_bytes(*dims) == 2 * one <= 5 << 30
        for f in (lib.qlka_abs_fwd_ws_bytes, lib.qlka_laplace_fwd_ws_bytes):
            assert f(*dims) == 2 * f(1, *dims[1:]) <= 5 << 30
    finally:
        lib.qlka_set_workspace_budget(prev)


@pytest.mark.parametrize("dims,msg", [
    ((1, 1, 8, 8, 129), "C (v.size(2)) must be in [1, 128]"),
    ((1, 1, 8, 8, 0), "C (v.size(2)) must be in [1, 128]"),
    ((1, 1, 131073, 8, 4), "N and M must be <= 131072"),
    ((1, 0, 8, 8, 4), "N, M and D must be > 0"),
    ((40000, 64, 1000, 1000, 4), "P*D*max(N,M) must fit int32"),
])
def test_validation_before_any_gpu_call(lib, dims, msg):
    P, D, N, M, C = dims
    dummy = ctypes.c_void_p(16)     # never dereferenced: validation fails first
    rc = lib.qlka_laplace_fwd(dummy, dummy, dummy, dummy, dummy, P, D, N, M, C, dummy, 1 << 40, None)
    assert rc == 1
    assert msg in lib.qlka_last_error().decode()
    rc = lib.qlka_abs_fwd(dummy, dummy, dummy, dummy, dummy, P, D, N, M, C, -1, dummy, 1 << 40, None)
    assert rc == 1


def test_path_and_workspace_errors(lib):
    dummy = ctypes.c_void_p(16)
    rc = lib.qlka_abs_fwd(dummy, dummy, dummy, dummy, dummy, 1, 1, 5000, 8, 4, 1, dummy, 1 << 40, None)
    assert rc == 1 and "fused path pinned but unavailable" in lib.qlka_last_error().decode()
    rc = lib.qlka_abs_fwd(dummy, dummy, dummy, dummy, dummy, 1, 1, 8, 8, 4, 2, dummy, 1 << 40, None)
    assert rc == 1 and "path must be -1 (auto), 0 (global) or 1 (fused)" in lib.qlka_last_error().decode()
    # a sort + walk shape (the dense route takes no workspace): the size check fails before any launch
    rc = lib.qlka_laplace_fwd(dummy, dummy, dummy, dummy, dummy, 1, 1, 800, 800, 4, dummy, 16, None)
    assert rc == 2 and "workspace too small" in lib.qlka_last_error().decode()
    rc = lib.qlka_laplace_fwd(None, dummy, dummy, dummy, dummy, 1, 1, 8, 8, 4, dummy, 1 << 40, None)
    assert rc == 1 and "non-null" in lib.qlka_last_error().decode()


def test_layer_workspace_and_validation(lib):
    dims = (1, 64, 16384, 16384, 64)                          # one p: one chunk, one copy
    op = lib.qlka_abs_fwd_ws_bytes(*dims)
    lap, riesz, bump = (lib.qlka_layer_fwd_ws_bytes(kind, *dims) for kind in (0, 1, 2))
    one_eval = 16384 * 64 * 4 + 16384 * 4                      # out_w + out_u of one op evaluation
    assert lap >= lib.qlka_laplace_fwd_ws_bytes(*dims) + one_eval
    assert riesz >= op + one_eval
    slab = 64 * 16384 * 64 * 4                                 # one p's contribution rows
    assert bump >= op + 2 * slab                               # three query sets walked at once: three slabs
    assert bump < 3 * op
    # without a foldable epilogue (C / 4 not a power of two) the three evaluations share one slab in turn
    odd = (1, 64, 16384, 16384, 63)
    assert lib.qlka_layer_fwd_ws_bytes(2, *odd) < 2 * lib.qlka_abs_fwd_ws_bytes(*odd)
    assert lib.qlka_layer_fwd_ws_bytes(3, *dims) == 0
    dummy = ctypes.c_void_p(16)     # never dereferenced: validation fails first
    rc = lib.qlka_layer_fwd(3, dummy, dummy, dummy, None, dummy, 1, 1, 8, 8, 4, dummy, 1 << 40, None)
    assert rc == 1 and "kind must be" in lib.qlka_last_error().decode()
    rc = lib.qlka_layer_fwd(2, dummy, dummy, dummy, None, dummy, 1, 1, 8, 8, 129, dummy, 1 << 40, None)
    assert rc == 1 and "C (v.size(2)) must be in [1, 128]" in lib.qlka_last_error().decode()
    rc = lib.qlka_layer_fwd(0, dummy, dummy, dummy, None, dummy, 1, 1, 8, 8, 4, dummy, 16, None)
    assert rc == 2 and "workspace too small" in lib.qlka_last_error().decode()
    rc = lib.qlka_layer_fwd(1, dummy, dummy, dummy, None, None, 1, 1, 8, 8, 4, dummy, 1 << 40, None)
    assert rc == 1 and "non-null" in lib.qlka_last_error().decode()
    rc = lib.qlka_layer_fwd_masked(0, dummy, dummy, dummy, None, dummy, 1, 1, 8, 8, 4, dummy, 1 << 40, None)
    assert rc == 1 and "keep must be non-null" in lib.qlka_last_error().decode()
    rc = lib.qlka_layer_fwd_masked(5, dummy, dummy, dummy, dummy, dummy, 1, 1, 8, 8, 4, dummy, 1 << 40, None)
    assert rc == 1 and "kind must be" in lib.qlka_last_error().decode()


def test_direct_cutoff_setter(lib):
    prev = lib.qlka_set_direct_max(0)
    try:
        assert prev == 512                       # the default
        assert lib.qlka_set_direct_max(100) == 0
        assert lib.qlka_set_direct_max(-1) < 0
        assert b"must be >= 0" in lib.qlka_last_error()
        assert lib.qlka_set_direct_max(prev) == 100   # a rejected value leaves the cutoff alone
    finally:
        lib.qlka_set_direct_max(prev)


def test_keep_sorts_entries_validate(lib):
    import ctypes
    kept = ctypes.c_int(7)
    # null sorted-array buffers are rejected before any launch, and *kept is cleared
    rc = lib.qlka_abs_fwd_keep(1, 1, 1, 1, None, 1, 1, 8, 8, 4, -1, None, None, None, None, None, ctypes.byref(kept),
                               None, 0, None)
    assert rc != 0 and kept.value == 0
    assert b"non-null" in lib.qlka_last_error()
    rc = lib.qlka_abs_bwd_sorted(1, 1, 1, 1, None, 1, 1, 1, 1, 1, 8, 8, 4, None, None, None, None, None, None, 0,
                                 None)
    assert rc != 0 and b"non-null" in lib.qlka_last_error()
    assert lib.qlka_abs_bwd_walks(12, 16384, 16384) == 1
    assert lib.qlka_abs_bwd_walks(512, 65, 65) == 0
    # the optional range states: ta and tb ([P*D][G+1][C+2] floats) and qb ([P*D][G] ints), 256-byte aligned each;
    # none where the backward takes the dense kernels or the merged walk (C <= 64, C % 4 == 0), which reads none
    def al(x):
        return (x + 255) // 256 * 256
    P, D, N, C, G = 12, 64, 16384, 62, 16384 // 64
    assert lib.qlka_abs_keep_state_bytes(P, D, N, N, C) == 2 * al(P * D * (G + 1) * (C + 2) * 4) + al(P * D * G * 4)
    assert lib.qlka_abs_keep_state_bytes(P, D, N, N, 64) == 0
    assert lib.qlka_abs_keep_state_bytes(P, D, N, N, 4) == 0
    assert lib.qlka_abs_keep_state_bytes(512, 32, 65, 65, 32) == 0
    # a handful of keys on either side: the dense route (the walk's segment totals would cost accuracy), also with the
    # cutoff at 0
    assert lib.qlka_abs_bwd_walks(12, 16384, 16) == 0 and lib.qlka_abs_bwd_walks(12, 16, 16384) == 0
    assert lib.qlka_abs_bwd_walks(12, 16384, 17) == 1
    prev = lib.qlka_set_direct_max(0)
    try:
        assert lib.qlka_abs_bwd_walks(12, 16384, 16) == 0
        assert lib.qlka_abs_bwd_walks(12, 16384, 17) == 1
    finally:
        lib.qlka_set_direct_max(prev)


def test_dense_keep_entries(lib):
    # the dense route keeps A (P*M rows of pad4(N) floats) where the forward and the backward both run dense, the
    # forward runs its tiled kernel (segments over 128) and A stays within 256 MB
    assert lib.qlka_abs_dense_keep_bytes(32, 64, 600, 600, 64) == 32 * 600 * 600 * 4
    assert lib.qlka_abs_dense_keep_bytes(3, 5, 301, 200, 33) == 3 * 200 * 304 * 4
    assert lib.qlka_abs_dense_keep_bytes(12, 64, 16384, 16384, 64) == 0      # walks
    assert lib.qlka_abs_dense_keep_bytes(12, 64, 600, 600, 64) == 0          # the backward walks at L = 600, P = 12
    assert lib.qlka_abs_dense_keep_bytes(512, 32, 65, 65, 32) == 0           # the one-workgroup kernel
    assert lib.qlka_abs_dense_keep_bytes(4096, 8, 512, 512, 8) == 0          # A over 256 MB
    # shapes where nothing is kept are rejected before any launch
    rc = lib.qlka_abs_fwd_dense_keep(1, 1, 1, 1, None, 1, 12, 64, 16384, 16384, 64, None)
    assert rc != 0 and b"not kept" in lib.qlka_last_error()
    rc = lib.qlka_abs_bwd_dense_kept(1, 1, 1, 1, None, 1, 1, 1, None, 32, 64, 600, 600, 64, None)
    assert rc != 0 and b"non-null" in lib.qlka_last_error()
