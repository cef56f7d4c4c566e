"""The C-ABI library (CPU only): it loads, exports every function include/lvattn.h declares, and rejects bad
arguments with a message before touching the GPU."""

import ctypes
import re
from pathlib import Path

import pytest

from lvattn import _capi

HEADER = Path(__file__).resolve().parents[1] / "include" / "lvattn.h"


def declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lv_\w+)\s*\(", text)))


def test_header_declares_the_path():
    names = declared()
    for name in ("lv_pack", "lv_store_kvcache", "lv_store_latents", "lv_paged_attention",
                 "lv_paged_attention_workspace_bytes", "lv_paged_attention_launch_info", "lv_merge_attn_states",
                 "lv_last_error", "lv_abi_version"):
        assert name in names


def test_library_exports_every_declared_symbol():
    lib = _capi.load()
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, f"declared in lvattn.h but not exported: {missing}"
    assert lib.lv_abi_version() == 9
    assert all(n in _capi._PROTOTYPES for n in declared()), "every declared function has a ctypes prototype"


def test_bad_arguments_raise_with_the_library_message():
    with pytest.raises(_capi.LvError, match="rows; 1 to 4096"):
        _capi.call("lv_pack", None, None, None, None, 0, 1, 16, 0, 0, *[None] * 10, 0, None)
    with pytest.raises(_capi.LvError, match="block_size must be positive"):
        _capi.call("lv_store_kvcache", None, None, 0, 0, 1, 1, 8, None, None, 0, 0, 0, 0, None, 2, None)
    with pytest.raises(_capi.LvError, match="head_dim 96"):
        _capi.call("lv_paged_attention", 1, 0, 0, 1, 1, 0, 0, 0, 16, 1, 0, None, 1, None, 1, 1, 8, 2, 96, 1.0, 1, 16,
                   1, 0, 0, None, 0, 0, 0, 0, 0, None)
    with pytest.raises(_capi.LvError, match="not bf16 or fp16"):
        _capi.call("lv_paged_attention", 1, 0, 0, 1, 1, 0, 0, 0, 16, 1, 0, None, 1, None, 1, 1, 8, 2, 64, 1.0, 1, 16,
                   1, 0, 0, None, 0, 0, 0, 0, 7, None)
    with pytest.raises(_capi.LvError, match="unknown schedule 5"):
        _capi.call("lv_paged_attention", 1, 0, 0, 1, 1, 0, 0, 0, 16, 1, 0, None, 1, None, 1, 1, 8, 2, 64, 1.0, 1, 16,
                   1, 0, 0, None, 0, 5, 0, 0, 0, None)
    with pytest.raises(_capi.LvError, match="cu_seqlens_ctx is null"):
        _capi.call("lv_varlen_context_attention", 1, 0, 0, 1, 0, 0, 1, 0, 0, 1, 1, 1, 0, 0, 1, 0, 0, None, 1, 16, 16,
                   192, 128, 1.0, 16, 1, 0, 0, None, 0, 0, 0, None)
    with pytest.raises(_capi.LvError, match="context keys, values and their strides must be 16-byte aligned"):
        _capi.call("lv_varlen_context_attention", 16, 0, 0, 16, 0, 0, 16, 0, 0, 16, 16, 17, 0, 0, 16, 0, 0, 16, 1, 16,
                   16, 192, 128, 1.0, 16, 16, 0, 0, None, 0, 0, 0, None)
    with pytest.raises(_capi.LvError, match="negative prompt_workgroups"):
        _capi.call("lv_paged_attention", 1, 0, 0, 1, 1, 0, 0, 0, 16, 1, 0, None, 1, None, 1, 1, 8, 2, 64, 1.0, 1, 16,
                   1, 0, 0, None, 0, 2, -1, 0, 0, None)


def test_workspace_query_sizes():
    # pure decode of one short row needs no split-K partials
    small = _capi.query("lv_paged_attention_workspace_bytes", 1, 1, 8, 2, 64, 64, 1)
    big = _capi.query("lv_paged_attention_workspace_bytes", 16, 16, 32, 8, 128, 131072, 1)
    assert small <= 512 and big > 1 << 20
    assert _capi.query("lv_paged_attention_workspace_bytes", 0, 0, 8, 2, 64, 64, 1) == 0


def test_the_static_workspace_refuses_a_step_that_needs_more():
    """lv_paged_attention_static sizes the step before it touches the GPU; a step whose work list and split-K
    partials exceed LV_STATIC_WORKSPACE_BYTES is refused with a message naming both sizes. (Arguments are fake
    non-null pointers: the call returns before using them.)"""
    # Split-K keeps a step's partials under 9 MiB at any context length; a step of 2^25 prompt tokens over one kv
    # head needs a work list of 2M items (16.8 MB) and still fits one launch.
    assert _capi.query("lv_paged_attention_workspace_bytes", 4096, 4096, 32, 8, 128, 1 << 30, 1) < 9 << 20
    assert _capi.query("lv_paged_attention_workspace_bytes", 4096, 4096, 32, 8, 128, (1 << 30) + 1, 1) == 0
    tokens = 1 << 25
    need = _capi.query("lv_paged_attention_workspace_bytes", 4096, tokens, 8, 1, 128, 1 << 20, 0)
    assert need > 16 << 20
    with pytest.raises(_capi.LvError, match=rf"needs {need} bytes of workspace; the static workspace holds 16777216"):
        _capi.call("lv_paged_attention_static", 16, 0, 0, 16, 16, 0, 0, 0, 256, 16, 0, 16, None, 16, 4096,
                   tokens, 8, 1, 128, 1.0, 64, 1 << 20, 16, 0, 0, 0, 0, 0, 0, None)


def test_the_launch_query_checks_its_shape_before_touching_the_gpu():
    """lv_paged_attention_launch_info applies the call's own shape checks first (a bad shape is refused with the
    call's message), and reports no kernels for a step without rows; neither case reads the device."""
    with pytest.raises(_capi.LvError, match="head_dim 96"):
        _capi.launch_info(4, 4, 8, 2, 96, 16, 64, 0, 1, 64, 0, 0, 0, 0)
    with pytest.raises(_capi.LvError, match="unknown schedule 7"):
        _capi.launch_info(4, 4, 8, 2, 64, 16, 64, 0, 1, 64, 7, 0, 0, 0)
    with pytest.raises(_capi.LvError, match="LV_ATTN_PROMPTS_ONLY needs cu_seqlens_q"):
        _capi.launch_info(4, 4, 8, 2, 64, 16, 64, 0, 1, 64, 0, 0, 2, 0)
    with pytest.raises(_capi.LvError, match="a step with prompts holds at most 4096 rows"):
        _capi.launch_info(5000, 9000, 8, 2, 64, 16, 64, 1, 8, 64, 0, 0, 0, 0)
    info = _capi.launch_info(0, 0, 8, 2, 64, 16, 64, 0, 1, 64, 0, 0, 0, 0)
    assert info["decode_kernel"] == info["prompt_kernel"] == "none"


def test_stores_and_merges_too_large_for_one_launch_are_refused():
    """Every launch counts the work-items along a grid dimension in 32 bits: a scatter of 2^31 - 1 tokens, a latent
    scatter of 2^25 tokens and a merge of 2^26 token rows are refused with a message before the GPU is touched (fake
    non-null, 16-byte-aligned pointers)."""
    big = (1 << 31) - 1
    with pytest.raises(_capi.LvError, match="store_kvcache: 2147483647 tokens need a grid larger than one launch"):
        _capi.call("lv_store_kvcache", 16, 16, 1024, 1024, big, 8, 128, 16, 16, 16 * 1024, 1024, 128, 16, 16, 2, None)
    with pytest.raises(_capi.LvError, match="store_latents: 33554432 tokens of 1152 bytes need a grid larger"):
        _capi.call("lv_store_latents", 16, 576, 1 << 25, 576, 16, 16, 2, None)
    with pytest.raises(_capi.LvError, match="merge_attn_states: 67108864 tokens x 1 heads need a grid larger"):
        _capi.call("lv_merge_attn_states", 16, 128, 128, 16, 128, 128, 16, 1, 1, 16, 128, 128, 16, 1, 1, 1 << 26, 1,
                   128, 0, None)


def test_a_key_bound_past_2_30_is_refused():
    """max_seqlen_k sizes the split-K grid in 32-bit counts: a bound above 2^30 keys is refused by the call (and sizes
    no workspace) before the GPU is touched."""
    with pytest.raises(_capi.LvError, match="max_seqlen_k 1073741825 is negative or above 2\\^30 keys"):
        _capi.call("lv_paged_attention", 16, 0, 0, 16, 16, 0, 0, 0, 256, 16, 0, None, 16, None, 5000, 5000, 32, 8, 128,
                   1.0, 1, (1 << 30) + 1, 16, 0, 0, 256, 1 << 40, 0, 0, 0, 0, None)


def test_a_step_too_large_for_one_launch_is_refused():
    """A step whose prompt grid would pass the 32-bit work-item count of one launch is refused with a message, by
    the call and by the launch query alike, before anything touches the GPU (fake non-null pointers)."""
    tokens = 1 << 29
    with pytest.raises(_capi.LvError, match="more than one launch holds"):
        _capi.launch_info(4096, tokens, 32, 8, 128, 256, 128, 1, 1 << 20, 1 << 20, 0, 0, 0, 0)
    with pytest.raises(_capi.LvError, match="more than one launch holds"):
        _capi.call("lv_paged_attention", 16, 0, 0, 16, 16, 0, 0, 0, 256, 16, 0, 16, None, 16, 4096, tokens, 32, 8, 128,
                   1.0, 1 << 20, 1 << 20, 16, 0, 0, 256, 1 << 40, 0, 0, 0, 0, None)


def test_a_varlen_call_too_large_for_one_launch_is_refused():
    """Attention over packed keys counts workgroups x threads against the same 32-bit limit: one row of up to
    2^31 - 1 queries over 8 kv heads needs 134M workgroups of 256 threads, refused before the GPU is touched (fake
    non-null pointers); both entry points share the check."""
    q_max = (1 << 31) - 1
    with pytest.raises(_capi.LvError, match="need 134217728 workgroups, more than one launch holds"):
        _capi.call("lv_varlen_attention", 16, 0, 0, 16, 0, 0, 16, 0, 0, 16, 16, 1, 8, 8, 128, 128, 1.0, 1, q_max, 16,
                   0, 0, None, 0, 0, 0, None)
    with pytest.raises(_capi.LvError, match="more than one launch holds"):
        _capi.call("lv_varlen_context_attention", 16, 0, 0, 16, 0, 0, 16, 0, 0, 16, 16, 16, 0, 0, 16, 0, 0, 16, 1, 16,
                   16, 192, 128, 1.0, q_max, 16, 0, 0, None, 0, 0, 0, None)


def test_token_strides_too_large_for_the_tile_offsets_are_refused():
    """Lanes address the rows of a 64-key tile with 32-bit offsets, computed as 24-bit products of key row and token
    stride: a cache or packed-key token stride of 2^23 elements (64 rows span 2^30 bytes) is refused by paged
    attention and by both packed-key entry points before the GPU is touched (fake non-null pointers)."""
    st = 1 << 23
    with pytest.raises(_capi.LvError, match="cache token stride 8388608 is negative or too large"):
        _capi.call("lv_paged_attention", 16, 0, 0, 16, 16, 0, st, 0, 256, 16, 0, None, 16, None, 1, 1, 32, 8, 128,
                   1.0, 1, 1024, 16, 0, 0, 256, 1 << 40, 0, 0, 0, 0, None)
    with pytest.raises(_capi.LvError, match="key token stride 8388608 or value token stride 0 is negative or too"):
        _capi.call("lv_varlen_attention", 16, 0, 0, 16, st, 0, 16, 0, 0, 16, 16, 1, 8, 8, 128, 128, 1.0, 1, 16, 16,
                   0, 0, None, 0, 0, 0, None)
    with pytest.raises(_capi.LvError, match="context token stride 0 or 8388608 is negative or too large"):
        _capi.call("lv_varlen_context_attention", 16, 0, 0, 16, 0, 0, 16, 0, 0, 16, 16, 16, 0, 0, 16, st, 0, 16, 1, 16,
                   16, 192, 128, 1.0, 16, 16, 0, 0, None, 0, 0, 0, None)
