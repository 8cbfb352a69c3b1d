"""CPU checks of the C ABI: the library loads, exports every symbol include/aegist_mixer.h
declares, rejects bad shapes with an error code and message before touching the device, and
hands out the same RoPE table the oracle uses. No kernel is launched here."""
import ctypes as C
import re
from pathlib import Path

import pytest
import torch

from conftest import ROOT
from oracle import mixer_ref as R

import aegist_mixer
from aegist_mixer import _lib

HEADER = ROOT / "include" / "aegist_mixer.h"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w]+\s*\*?\s*(aegist_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    names = declared_symbols()
    assert len(names) >= 25
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, f"not exported: {missing}"
    # and the ctypes table covers the header exactly
    assert sorted(_lib.SIGNATURES) == names


def test_version_and_no_error_initially():
    assert b"gfx950" in _lib.lib().aegist_version()


def test_rope_table_matches_oracle_bitwise():
    for rd, theta in [(64, 1e7), (32, 1e4), (256, 5e5)]:
        ours = aegist_mixer.ops.rope_inv_freq(rd, theta)
        assert torch.equal(ours, R.rope_inv_freq(rd, theta))


def test_rope_rejects_odd_dim():
    buf = (C.c_float * 8)()
    rc = _lib.lib().aegist_rope_inv_freq(buf, 7, 1e4)
    assert rc == -1 and "even" in _lib.last_error()


@pytest.mark.parametrize("hk,hv", [(16, 24), (16, 48), (3, 5)])
def test_decode_step_rejects_head_ratio(hk, hv):
    rc = _lib.lib().aegist_delta_decode_step(None, 1, None, None, None, None, None, None, 0, 4, hk, hv,
                                             0.088, 1e-6, None)
    assert rc == -1 and "HV" in _lib.last_error()


def test_decode_step_rejects_bad_dtype():
    rc = _lib.lib().aegist_delta_decode_step(None, 7, None, None, None, None, None, None, 0, 4, 16, 32,
                                             0.088, 1e-6, None)
    assert rc == -3


def test_attention_decode_rejects_shapes():
    L = _lib.lib()
    args = [None, None, None, 1, None, None, None, None, None, 0]
    rc = L.aegist_attention_decode(*args, 1, 16, 2, 128, 64, 10, 100, 1e-6, 1e7, None, 0, None)
    assert rc == -1 and "256" in _lib.last_error()
    rc = L.aegist_attention_decode(*args, 1, 16, 3, 256, 64, 10, 100, 1e-6, 1e7, None, 0, None)
    assert rc == -1
    rc = L.aegist_attention_decode(*args, 1, 16, 2, 256, 64, 100, 100, 1e-6, 1e7, None, 0, None)
    assert rc == -1 and "cap" in _lib.last_error()
    rc = L.aegist_attention_decode(*args, 1, 16, 2, 256, 64, 10, 100, 1e-6, 1e7, None, 0, None)
    assert rc == -2  # workspace missing


def test_workspace_queries_are_host_only():
    L = _lib.lib()
    a = L.aegist_attention_decode_workspace_bytes(32, 16, 2, 131073)
    b = L.aegist_attention_decode_workspace_bytes(1, 16, 2, 4097)
    assert a > 0 and b > 0 and a % 256 == 0
    if hasattr(L, "aegist_delta_chunked_workspace_bytes"):
        assert L.aegist_delta_chunked_workspace_bytes(1, 8192, 32) > 0


def test_engine_mirrors_reject_shapes():
    L = _lib.lib()
    assert L.aegist_delta_scan(None, None, None, None, 4, 8191, 16, 32, None) == -1
    assert L.aegist_l2norm_heads(None, 4, 100, 16, 128, 1.0, 1e-6, None) == -1


def test_linear_rejects_shapes_and_dtypes():
    L = _lib.lib()
    # K % 16 != 0
    assert L.aegist_linear(None, 0, 24, None, 2, None, None, 8, 2, 8, 24, 0, None) == -1
    assert b"multiple of 16" in L.aegist_last_error()
    # ldy < N
    assert L.aegist_linear(None, 0, 32, None, 2, None, None, 4, 2, 8, 32, 0, None) == -1
    # unsupported weight dtype (fp32 weights are not a QLinear form)
    assert L.aegist_linear(None, 0, 32, None, 0, None, None, 8, 2, 8, 32, 0, None) == -3
    # the engine argument lists validate the same way
    assert L.aegist_gemv_i8(None, None, None, None, 8, 24, 0, None) == -1
    assert L.aegist_gemm_i8(None, None, None, None, 3, 8, 40, 0, None) == -1
    # empty outputs are a no-op
    assert L.aegist_gemm_i8(None, None, None, None, 0, 8, 32, 0, None) == 0


def test_linear_multi_rejects_counts():
    L = _lib.lib()
    arr = (C.c_void_p * 5)()
    lds = (C.c_longlong * 5)(*([8] * 5))
    ns = (C.c_int * 5)(*([8] * 5))
    for n in (0, 5):
        assert L.aegist_linear_multi(None, 0, 32, 2, n, arr, None, arr, lds, ns, 2, 32, 0, None) == -1
    assert L.aegist_linear_multi(None, 0, 32, 2, 1, None, None, arr, lds, ns, 2, 32, 0, None) == -1


def test_stack_state_entry_points_reject_null_handle():
    L = _lib.lib()
    assert L.aegist_stack_snapshot(None, None) == -1
    assert L.aegist_stack_crop(None, 3, None) == -1
    assert L.aegist_stack_state_bytes(None, 3) == 0
    assert L.aegist_stack_save_state(None, 0, None, 0, None) == -1
    assert L.aegist_stack_load_state(None, 0, 1, None, 0, None) == -1


def test_indexer_entry_points_reject_shapes():
    L = _lib.lib()
    # the indexer head dim must be 128
    assert L.aegist_idx_prep(None, None, None, None, 1, 4, 64, 64, 0, 1e-6, 1e7, None) == -1
    assert L.aegist_idx_blocks(None, None, None, 0, 1, 4, 64, 64, 1e-6, 1e7, None) == -1
    assert L.aegist_idx_scores(None, None, None, 1, 4, 64, 0, 4, 8, None) == -1
    # odd rotary dim
    assert L.aegist_idx_prep(None, None, None, None, 1, 4, 128, 63, 0, 1e-6, 1e7, None) == -1
    # nbmax below the number of complete blocks
    assert L.aegist_idx_select(None, None, None, 1, 16, 4, 100, 10, None) == -1
    # top / R must be positive; list attention needs H % KV == 0 and positions inside the cache
    assert L.aegist_idx_select(None, None, None, 1, 0, 4, 0, 8, None) == -1
    assert L.aegist_attention_gated_list(None, None, None, None, None, 1, 6, 4, 0, 8, 1.0, None, None, 4, 4,
                                         None) == -1
    assert L.aegist_attention_gated_list(None, None, None, None, None, 2, 16, 2, 7, 8, 1.0, None, None, 4, 4,
                                         None) == -1
    assert L.aegist_gated_norm2(None, None, None, None, 1, 0, 128, 1e-6, 1, None) == -1
    # empty inputs are a no-op
    assert L.aegist_idx_select(None, None, None, 0, 16, 4, 0, 8, None) == 0


def test_reference_signature_mirrors_need_a_bound_workspace():
    """Mirrors whose reference signature has no workspace argument never allocate: with nothing
    bound they return AEGIST_ERR_WORKSPACE (checked before any launch) and say how to bind one."""
    L = _lib.lib()
    assert L.aegist_attention_gated_workspace_bytes(1, 16, 2, 4096) > 0
    assert L.aegist_attention_gated_workspace_bytes(5, 16, 2, 4096) == 0  # prefill uses no scratch
    assert L.aegist_delta_scan_workspace_bytes(63, 16, 32) == 0
    assert L.aegist_delta_scan_workspace_bytes(64, 16, 32) > 0
    assert L.aegist_router_topk_workspace_bytes(4, 256) == 4 * 256 * 4
    rc = L.aegist_attention_gated(None, None, None, None, None, 1, 16, 2, 4096, 8192, 0.0625, None)
    assert rc == -2 and "aegist_bind_workspace" in _lib.last_error()
    C_ = 2 * 16 * 128 + 32 * 128
    assert L.aegist_delta_scan(None, None, None, None, 64, C_, 16, 32, None) == -2
    assert L.aegist_router_topk(None, None, None, None, 4, 256, 256, 8, None) == -2
    # an explicit workspace that is too small or misaligned is refused the same way
    assert L.aegist_delta_scan_ws(None, None, None, None, 64, C_, 16, 32, None, 0, None) == -2
    assert L.aegist_attention_gated_ws(None, None, None, None, None, 1, 16, 2, 4096, 8192, 0.0625, 8, 1 << 30,
                                       None) == -2
