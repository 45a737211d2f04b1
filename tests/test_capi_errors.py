"""The C ABI's argument checks without a GPU: malformed views and arguments are
rejected with LOGKV_EINVAL (or a negative size) and a message in logkv_last_error,
before anything is launched. Every case here fails a check that precedes the first
HIP call of its entry point; the pointers are never dereferenced.

The fake device addresses are only safe while no kernel can launch, so the module
runs only where no HIP device is visible (the CPU suite); where a device is
visible the same checks are exercised through real tensors by the GPU tests."""

import ctypes as C

import pytest
import torch

from logkv_amd import _lib

pytestmark = pytest.mark.skipif(torch.cuda.is_available(),
                                reason="fake device addresses are only passed where no HIP device is visible")

FAKE = 0x10000   # a 64 KiB-aligned address that the checks accept and nothing reads


@pytest.fixture(scope="module")
def lib():
    return _lib.lib()


def last_error(lib):
    return (lib.logkv_last_error() or b"").decode()


def ladder(**over):
    v = _lib.LadderView()
    for name, _ in _lib.LadderView._fields_[:16]:
        setattr(v, name, FAKE)
    v.n_batch, v.n_groups, v.k_max, v.levels, v.slots, v.dk, v.dv = 1, 2, 4, 5, 8, 128, 128
    for k, x in over.items():
        setattr(v, k, x)
    return v


def test_valid_ladder_view_sizes_a_workspace(lib):
    assert lib.logkv_route_workspace_bytes(C.byref(ladder()), 64, 0) > 0


@pytest.mark.parametrize("over,message", [
    ({"k_max": 0}, "cluster count"),
    ({"k_max": 33}, "cluster count"),
    ({"slots": 1}, "slots per level"),
    ({"slots": 40000}, "slots per level"),
    ({"levels": 0}, "levels"),
    ({"dk": 6}, "multiples of 4"),
    ({"dv": 0}, "multiples of 4"),
    ({"centroid": 0}, "NULL buffer"),
    ({"level_k": FAKE + 8}, "16-byte aligned"),
    ({"n_batch": 0}, "batch and groups"),
])
def test_malformed_ladder_view_is_rejected(lib, over, message):
    assert lib.logkv_route_workspace_bytes(C.byref(ladder(**over)), 64, 0) < 0
    assert message in last_error(lib)


def test_null_views_and_short_workspaces_are_rejected(lib):
    params = _lib.RouteParams(1.0, 1.0, 1.0, 0, 0)
    rows = _lib.RowsView()
    rows.k = rows.v = rows.pos = FAKE
    rows.k_sb = rows.v_sb = 2 * 64 * 128
    rows.k_sg = rows.v_sg = 64 * 128
    rows.k_st = rows.v_st = 128
    rows.pos_sb, rows.tokens = 64, 64
    assert lib.logkv_attach_assign(None, C.byref(rows), C.byref(params), FAKE, 1 << 30, FAKE, FAKE,
                                   None) == _lib.LOGKV_EINVAL
    assert "NULL" in last_error(lib)
    # A workspace one byte short of the size the library asks for.
    need = lib.logkv_route_workspace_bytes(C.byref(ladder()), 64, 0)
    assert lib.logkv_route_commit(C.byref(ladder()), C.byref(rows), C.byref(params), FAKE, need - 1,
                                  None, None, None) == _lib.LOGKV_EINVAL
    assert "smaller than" in last_error(lib)
    # Rows that are not 8-byte aligned.
    rows.k_st = 130
    assert lib.logkv_route_commit(C.byref(ladder()), C.byref(rows), C.byref(params), FAKE, need,
                                  None, None, None) == _lib.LOGKV_EINVAL
    assert "aligned" in last_error(lib)


def test_attention_arguments_are_checked(lib):
    a = _lib.AttentionArgs()
    a.q, a.k, a.v, a.out = FAKE, FAKE, FAKE, FAKE
    a.n_batch, a.n_heads, a.n_groups, a.tq, a.dk, a.dv, a.dim = 1, 4, 2, 1, 128, 128, 136
    a.cap, a.tail, a.scale = 64, 1, 0.088
    a.q_sb, a.q_sh, a.q_st = 4 * 128, 128, 128
    a.o_sb, a.o_sh, a.o_st = 4 * 128, 128, 128
    table = (C.c_int32 * 4)()
    need = lib.logkv_attention_workspace_bytes(C.byref(a))
    assert need > 0

    def decode(**over):
        for k, x in over.items():
            setattr(a, k, x)
        return lib.logkv_decode_attention(C.byref(a), table, 4, FAKE, need, None)

    assert decode(dim=128) == _lib.LOGKV_EINVAL and "packed width" in last_error(lib)   # no room for the bias
    assert decode(dim=136, n_heads=3) == _lib.LOGKV_EINVAL and "multiple of groups" in last_error(lib)
    assert decode(n_heads=4, tq=9) == _lib.LOGKV_EINVAL and "queries per KV group" in last_error(lib)
    assert decode(tq=1, causal_tail=2) == _lib.LOGKV_EINVAL and "causal_tail" in last_error(lib)
    assert decode(causal_tail=0, n_batch=0) == _lib.LOGKV_EINVAL and "n_batch" in last_error(lib)
    assert decode(n_batch=1, cap=0, tail=0) == _lib.LOGKV_EINVAL and "cap" in last_error(lib)
    assert decode(cap=64, tail=1, k=FAKE + 8) == _lib.LOGKV_EINVAL and "16-byte aligned" in last_error(lib)
    assert decode(k=FAKE, v=FAKE + 8) == _lib.LOGKV_EINVAL and "16-byte aligned" in last_error(lib)
    a.v = FAKE
    a.causal_tail = 0
    assert lib.logkv_decode_attention(C.byref(a), table, 4, FAKE, need - 1, None) == _lib.LOGKV_EINVAL
    assert "workspace too small" in last_error(lib)
    assert lib.logkv_decode_attention(C.byref(a), None, 4, FAKE, need, None) == _lib.LOGKV_EINVAL
