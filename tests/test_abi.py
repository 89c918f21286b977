"""The C ABI library: loads on a machine without a GPU, exports every entry
point include/nanokv.h declares, and rejects bad arguments before touching
the device (no compute calls here)."""

import ctypes
import os
import re

import pytest

from nanokv_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "nanokv.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = {}
    for m in re.finditer(r"\b(?:int|int64_t|const char\s*\*)\s+(nkv_\w+)\s*\(([^)]*)\)\s*;", text):
        args = [a.strip() for a in m.group(2).split(",") if a.strip() and a.strip() != "void"]
        decls[m.group(1)] = len(args)
    return decls


def test_library_loads_and_reports_abi_version():
    lib = _lib.load()
    assert lib.nkv_abi_version() == _lib.ABI_VERSION


def test_every_declared_entry_point_is_exported_with_matching_arity():
    lib = _lib.load()
    decls = _declared()
    assert {"nkv_select", "nkv_attend", "nkv_store_chunk", "nkv_build_reps",
            "nkv_recent_update", "nkv_query_summaries"} <= set(decls)
    for name, nargs in decls.items():
        assert hasattr(lib, name), f"{name} not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
        assert len(_lib.SIGNATURES[name][1]) == nargs, f"{name}: {nargs} args declared"


def test_bad_arguments_are_rejected_before_any_device_work():
    lib = _lib.load()
    rc = lib.nkv_select(None, 0, 1, None, 0, 1, 0, 1, None, 0, 32, 0, None, None, None, None, None)
    assert rc == _lib.NKV_ERR_ARG
    assert b"store descriptor is NULL" in lib.nkv_last_error()
    st = _lib.NkvStore()
    st.head_dim, st.block_size = 64, 64
    rc = lib.nkv_attend(ctypes.byref(st), 0, 1, None, 0, 1, None, None, 0, 0, -1, None, 0, 0,
                        None, 0, 0, 0, 0, 0, 1.0, 1, None, None, None)
    assert rc == _lib.NKV_ERR_UNSUPPORTED
    with pytest.raises(ValueError, match="head_dim"):
        _lib.check(rc, "attend")
    rc = lib.nkv_query_summaries(None, 0, 1, 8, 32, 128, 1, None, 0, None)
    assert rc == _lib.NKV_ERR_ARG


def test_prefill_entry_rejects_bad_arguments_without_device_work():
    lib = _lib.load()
    st = _lib.NkvStore()
    st.num_layers, st.num_heads, st.num_kv_heads = 1, 32, 8
    st.head_dim, st.block_size, st.r, st.cap_blocks = 128, 64, 4, 16
    st.sink_tokens, st.recent_tokens, st.kv_format = 64, 512, 0
    dummy = ctypes.c_void_p(16)   # never dereferenced: every call below fails validation
    st.hist_k = st.hist_v = st.reps = dummy
    st.sink_k = st.sink_v = st.recent_k = st.recent_v = dummy
    # q NULL
    rc = lib.nkv_prefill_attend(ctypes.byref(st), 0, 1, None, 0, 64, dummy, dummy, 0, None, 0, 0,
                                None, 0, 0, 0, 0, 0, 1.0, 1, None, dummy, None)
    assert rc == _lib.NKV_ERR_ARG and b"nkv_prefill_attend" in lib.nkv_last_error()
    # recent range beyond the ring
    rc = lib.nkv_prefill_attend(ctypes.byref(st), 0, 1, dummy, 0, 64, dummy, dummy, 0, None, 0, 0,
                                None, 0, 0, 0, 500, 100, 1.0, 1, None, dummy, None)
    assert rc == _lib.NKV_ERR_ARG and b"recent range" in lib.nkv_last_error()
    # chunk K/V missing
    rc = lib.nkv_prefill_attend(ctypes.byref(st), 0, 1, dummy, 0, 64, None, None, 0, None, 0, 0,
                                None, 0, 0, 0, 0, 0, 1.0, 1, None, dummy, None)
    assert rc == _lib.NKV_ERR_ARG and b"k_new/v_new" in lib.nkv_last_error()
    # GQA group size that does not divide the 128-column query tile
    st.num_heads, st.num_kv_heads = 24, 8
    rc = lib.nkv_prefill_attend(ctypes.byref(st), 0, 1, dummy, 0, 64, dummy, dummy, 0, None, 0, 0,
                                None, 0, 0, 0, 0, 0, 1.0, 1, None, dummy, None)
    assert rc == _lib.NKV_ERR_UNSUPPORTED


def test_decode_step_rejects_bad_arguments_without_device_work():
    lib = _lib.load()
    st = _lib.NkvStore()
    st.num_layers, st.num_heads, st.num_kv_heads = 4, 32, 8
    st.head_dim, st.block_size, st.r, st.cap_blocks = 128, 64, 4, 16
    st.sink_tokens, st.recent_tokens, st.kv_format = 64, 512, 0
    dummy = ctypes.c_void_p(16)   # never dereferenced: every call below fails validation
    st.hist_k = st.hist_v = st.reps = dummy
    st.sink_k = st.sink_v = st.recent_k = st.recent_v = dummy
    streams = (ctypes.c_void_p * 2)(None, None)

    def call(nstreams=2, streams_arr=streams, n_hist=32, q=dummy, partial=dummy, splits=3):
        return lib.nkv_decode_step(ctypes.byref(st), 0, 4, q, dummy, dummy, 16, dummy, 1, 32, n_hist,
                                   64, 0, 1, 0, 511, 1.0, splits, dummy, dummy, partial, dummy,
                                   nstreams, streams_arr)

    assert call(nstreams=0) == _lib.NKV_ERR_ARG and b"nstreams" in lib.nkv_last_error()
    assert call(nstreams=9) == _lib.NKV_ERR_ARG and b"nstreams" in lib.nkv_last_error()
    assert call(streams_arr=None) == _lib.NKV_ERR_ARG and b"streams is NULL" in lib.nkv_last_error()
    assert call(q=None) == _lib.NKV_ERR_ARG and b"non-NULL" in lib.nkv_last_error()
    assert call(n_hist=33) == _lib.NKV_ERR_ARG and b"n_hist" in lib.nkv_last_error()
    assert call(n_hist=0) == _lib.NKV_ERR_ARG and b"n_hist" in lib.nkv_last_error()
    assert call(partial=None) == _lib.NKV_ERR_ARG and b"partial_ws" in lib.nkv_last_error()
    # one attention workspace per range, sized for the largest range
    per = lib.nkv_attend_workspace_floats(2, 8, 32, 1, 3)
    assert lib.nkv_decode_step_workspace_floats(4, 8, 32, 3, 2) == 2 * per
    assert lib.nkv_decode_step_workspace_floats(4, 8, 32, 3, 0) == 0


def test_select_union_rejects_bad_arguments_without_device_work():
    lib = _lib.load()
    d = ctypes.c_void_p(16)   # never dereferenced: every call below fails validation
    assert lib.nkv_select_union(None, 1, 6, 32, 32, 192, d, d, d, None) == _lib.NKV_ERR_ARG
    assert lib.nkv_select_union(d, 1, 0, 32, 32, 192, d, d, d, None) == _lib.NKV_ERR_ARG
    assert lib.nkv_select_union(d, 1, 17, 32, 32, 544, d, d, d, None) == _lib.NKV_ERR_ARG
    assert lib.nkv_select_union(d, 1, 6, 32, 33, 198, d, d, d, None) == _lib.NKV_ERR_ARG
    assert b"k_eff" in lib.nkv_last_error()
    assert lib.nkv_select_union(d, 1, 6, 32, 32, 191, d, d, d, None) == _lib.NKV_ERR_ARG
    assert b"umax" in lib.nkv_last_error()
    assert lib.nkv_select_union(d, 1, 16, 512, 512, 8192, d, d, d, None) == _lib.NKV_ERR_UNSUPPORTED


def test_attend_rejects_a_short_allowed_layer_stride():
    lib = _lib.load()
    st = _lib.NkvStore()
    st.num_layers, st.num_heads, st.num_kv_heads = 2, 32, 8
    st.head_dim, st.block_size, st.r, st.cap_blocks = 128, 64, 4, 16
    st.sink_tokens, st.recent_tokens, st.kv_format = 64, 512, 0
    d = ctypes.c_void_p(16)   # never dereferenced: the call fails validation
    st.hist_k = st.hist_v = st.reps = d
    st.sink_k = st.sink_v = st.recent_k = st.recent_v = d
    # tq = 6 queries x n_hist = 10 blocks need a per-layer stride >= 60
    rc = lib.nkv_attend(ctypes.byref(st), 0, 2, d, 6 * 32 * 128, 6, d, d, 6 * 8 * 128, 6, -1, d, 10, 10,
                        d, 59, 64, 0, 0, 511, 1.0, 1, None, d, None)
    assert rc == _lib.NKV_ERR_ARG and b"allowed_layer_stride" in lib.nkv_last_error()


def test_host_device_pointer_rejects_null_without_device_work():
    lib = _lib.load()
    out = ctypes.c_void_p(1234)
    assert lib.nkv_host_device_pointer(None, ctypes.byref(out)) == _lib.NKV_ERR_ARG
    assert b"non-NULL" in lib.nkv_last_error()
    assert lib.nkv_host_device_pointer(ctypes.c_void_p(8), None) == _lib.NKV_ERR_ARG


def test_model_ops_reject_bad_sizes_without_device_work():
    lib = _lib.load()
    fake = ctypes.c_void_p(256)     # never dereferenced: the size checks come first
    assert lib.nkv_rmsnorm(fake, None, fake, fake, None, 1, 12, 1e-6, None) == _lib.NKV_ERR_ARG
    assert b"multiple of 8" in lib.nkv_last_error()
    assert lib.nkv_rmsnorm(fake, None, fake, fake, None, 1, 16384, 1e-6, None) == _lib.NKV_ERR_ARG
    assert lib.nkv_rmsnorm(fake, None, fake, fake, None, 0, 64, 1e-6, None) == _lib.NKV_ERR_ARG
    assert lib.nkv_rmsnorm(ctypes.c_void_p(258), None, fake, fake, None, 1, 64, 1e-6, None) == _lib.NKV_ERR_ARG
    assert b"aligned" in lib.nkv_last_error()
    assert lib.nkv_silu_mul(fake, fake, 1, 12, None) == _lib.NKV_ERR_ARG
    assert lib.nkv_silu_mul(None, fake, 1, 16, None) == _lib.NKV_ERR_ARG
    assert lib.nkv_qk_norm_rope(fake, 0, 32, 8, fake, fake, fake, fake, 10, fake, 1e-6, fake, fake, fake,
                                None) == _lib.NKV_ERR_ARG
    assert lib.nkv_qk_norm_rope(None, 1, 32, 8, fake, fake, fake, fake, 10, fake, 1e-6, fake, fake, fake,
                                None) == _lib.NKV_ERR_ARG


def test_packed_attention_rejects_bad_arguments_without_device_work():
    lib = _lib.load()
    d = ctypes.c_void_p(256)    # never dereferenced: the checks come first
    assert lib.nkv_attend_packed(24, 8, d, 4, d, d, 64, 0, None, 1.0, 1, None, d, None) == _lib.NKV_ERR_UNSUPPORTED
    assert lib.nkv_attend_packed(32, 7, d, 4, d, d, 64, 0, None, 1.0, 1, None, d, None) == _lib.NKV_ERR_ARG
    assert lib.nkv_attend_packed(32, 8, None, 4, d, d, 64, 0, None, 1.0, 1, None, d, None) == _lib.NKV_ERR_ARG
    assert lib.nkv_attend_packed(32, 8, d, 0, d, d, 64, 0, None, 1.0, 1, None, d, None) == _lib.NKV_ERR_ARG
    assert lib.nkv_attend_packed(32, 8, d, 4, d, d, 0, 0, None, 1.0, 1, None, d, None) == _lib.NKV_ERR_ARG
    assert lib.nkv_attend_packed(32, 8, d, 4, d, d, 64, -1, None, 1.0, 1, None, d, None) == _lib.NKV_ERR_ARG
    assert b"causal_from" in lib.nkv_last_error()
    assert lib.nkv_attend_packed(32, 8, d, 4, d, d, 64, 0, None, 1.0, 3, None, d, None) == _lib.NKV_ERR_ARG
    assert b"partial_ws" in lib.nkv_last_error()
    # the workspace follows the kernel choice: few-query rows (tq * G <= 16) vs query tiles
    assert lib.nkv_attend_packed_workspace_floats(32, 8, 4, 1) == 0
    assert lib.nkv_attend_packed_workspace_floats(32, 8, 4, 3) == lib.nkv_attend_workspace_floats(1, 8, 32, 4, 3)
    assert lib.nkv_attend_packed_workspace_floats(32, 8, 256, 3) == lib.nkv_prefill_workspace_floats(1, 8, 32, 256, 3)


def test_noalloc_decode_step_rejects_sizes_beyond_its_scratch_without_device_work():
    lib = _lib.load()
    st = _lib.NkvStore()
    st.num_layers, st.num_heads, st.num_kv_heads = 64, 32, 8
    st.head_dim, st.block_size, st.r, st.cap_blocks = 128, 64, 4, 8192
    st.sink_tokens, st.recent_tokens, st.kv_format = 64, 512, 0
    d = ctypes.c_void_p(256)    # never dereferenced: the size checks come first
    st.hist_k = st.hist_v = st.reps = d
    st.sink_k = st.sink_v = st.recent_k = st.recent_v = d

    def call(nl, nblocks, splits):
        return lib.nkv_decode_step_noalloc(ctypes.byref(st), 0, nl, d, d, d, nblocks, d, 1, 32, 32, 64, 0, 1, 0,
                                           511, 1.0, splits, d, d, None)

    # 64 layers x 4097 blocks = 262208 score keys > 262144
    assert call(64, 4097, 1) == _lib.NKV_ERR_ARG and b"score keys" in lib.nkv_last_error()
    # 36 layers x 8 heads x 7 splits of 16 x 130 floats = 4193280 > 3932160
    assert call(36, 512, 7) == _lib.NKV_ERR_ARG and b"split partials" in lib.nkv_last_error()
    # splits 0 is the stream form; below 0 or above 64 is refused
    assert call(36, 512, -1) == _lib.NKV_ERR_ARG and call(36, 512, 65) == _lib.NKV_ERR_ARG
    with pytest.raises(ValueError, match="score keys"):
        _lib.check(call(64, 4097, 1), "decode_step_noalloc")
