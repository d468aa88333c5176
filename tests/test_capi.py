"""The C-ABI library loads without a GPU, exports every entry point that
include/*.h declares, and its host-only logic works (no compute calls)."""
import ctypes as C
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")


def declared_symbols():
    names = set()
    for name in os.listdir(INCLUDE):
        if name.endswith(".h"):
            text = open(os.path.join(INCLUDE, name)).read()
            names.update(re.findall(r"\b(sa_hip_\w+)\s*\(", text))
    return sorted(names)


def test_header_declares_entry_points():
    syms = declared_symbols()
    assert "sa_hip_sparse_decode_attention" in syms and len(syms) >= 15


def test_library_exports_every_declared_symbol():
    import solidattention_amd as sa
    L = C.CDLL(sa.LIB_PATH)
    missing = [s for s in declared_symbols() if not hasattr(L, s)]
    assert not missing, missing
    # and the binding table covers them
    assert set(declared_symbols()) <= set(sa.EXPORTS)


def test_host_only_queries():
    import solidattention_amd as sa
    L = sa.lib()
    assert L.sa_hip_abi_version() == 1
    # workspace: batch * kv_heads * splits * group * (head_dim + 4) floats
    assert L.sa_hip_attention_workspace_bytes(64, 16, 8, 128, 4) == 64 * 8 * 4 * 2 * 132 * 4
    assert L.sa_hip_attention_workspace_bytes(64, 16, 8, 128, 1) == 0
    s = L.sa_hip_attention_default_splits(64, 8, 66)
    assert 1 <= s <= 64
    # resident workgroups per CU (256 CUs off the GPU): two for 1-2 query
    # heads per KV head, one 8-wave for 4, one 4-wave for 8; at least ~4
    # pages per wave
    assert L.sa_hip_attention_splits_for(64, 16, 8, 66) == 1 == s
    assert L.sa_hip_attention_splits_for(32, 32, 8, 66) == 1
    assert L.sa_hip_attention_splits_for(32, 16, 8, 66) == 2
    assert L.sa_hip_attention_splits_for(8, 32, 8, 66) == 2
    assert L.sa_hip_attention_splits_for(1, 64, 8, 1000) == 32
    assert L.sa_hip_attention_splits_for(1, 32, 8, 1 << 20) == 32


def test_compare_prediction_matches_oracle_on_p10(oracle_lib):
    import solidattention_amd as sa
    O = oracle_lib
    history = [O.oracle_blocks(0, layer) for layer in range(28)]
    misses_total = 0
    for step in range(16):
        for layer in range(28):
            oracle_set = O.oracle_blocks(step, layer)
            hits, misses, slots = sa.compare_prediction(history[layer], oracle_set)
            st, ohits, omisses, oslots = O.compare_prediction(history[layer], oracle_set)
            assert (hits, misses, slots) == (ohits, omisses, oslots)
            misses_total += len(misses)
            history[layer] = oracle_set
    assert misses_total == 346


def test_compare_prediction_cardinality_error():
    import solidattention_amd as sa
    with pytest.raises(sa.SaHipError, match="cardinality"):
        sa.compare_prediction([0, 0, 2, 15], [0, 1, 2, 15])


def test_contiguous_attention_head_dims():
    """head_dim 128 takes the paged kernel's workspace; other multiples of 8
    up to 512 the any-head_dim kernel's (records of head_dim + 2 floats per
    split and query head, none for a single split); the rest are refused
    before any launch."""
    import solidattention_amd as sa
    L = sa.lib()
    assert L.sa_hip_contiguous_workspace_bytes(100, 16, 8, 64) == 0  # one split below 512 tokens
    n = L.sa_hip_contiguous_workspace_bytes(40000, 16, 8, 64)  # 256 CUs off the GPU: 64 splits
    assert n == 8 * 64 * 2 * 66 * 4
    assert L.sa_hip_contiguous_workspace_bytes(40000, 16, 8, 100) == 0
    p = C.c_void_p(16)
    for d, hq, hkv, what in ((100, 16, 8, b"head_dim 100"), (1024, 16, 8, b"head_dim 1024"),
                             (64, 24, 8, b"24/8")):
        rc = L.sa_hip_attention_contiguous(p, p, 100, hq, hkv, d, C.c_float(1.0), p, None, 0, None)
        assert rc == -1 and what in L.sa_hip_last_error()


def test_invalid_arguments_fail_before_any_launch():
    """Argument validation returns SA_HIP_EINVAL with a message and launches
    nothing (safe without a GPU)."""
    import solidattention_amd as sa
    L = sa.lib()
    kv = sa.PagedKVStruct()
    # the paged path takes 128 or another multiple of 8 up to 512; the
    # chunked attention 128 only
    for d in (100, 1024, 0):
        kv.head_dim = d
        rc = L.sa_hip_sparse_decode_attention(C.byref(kv), None, None, None, 1, 1, C.c_float(1.0), None, None, 0, 1,
                                              None, None)
        assert rc == -1 and b"head_dim %d" % d in L.sa_hip_last_error()
    kv.head_dim = 64
    rc = L.sa_hip_sparse_decode_attention_chunked(C.byref(kv), None, None, None, 1, 1, C.c_float(1.0), None, None,
                                                  0, 2, 4, None, None)
    assert rc == -1 and b"head_dim 64" in L.sa_hip_last_error()
    kv.head_dim, kv.query_heads, kv.kv_heads = 128, 12, 8
    rc = L.sa_hip_score_select(C.byref(kv), None, None, None, None, None, None, None)
    assert rc == -1 and b"GQA" in L.sa_hip_last_error()
    p = sa.SelectParamsStruct(8, 4, 3, 2, 4)
    kv.query_heads = 16
    kv.batch, kv.table_stride, kv.num_pages = 1, 4, 4
    kv.pool = kv.block_table = kv.seq_len = kv.sealed = kv.reps = 16
    kv.rep_heads, kv.rep_stride = 8, 4
    rc = L.sa_hip_score_select(C.byref(kv), C.c_void_p(16), C.byref(p), C.c_void_p(16), C.c_void_p(16), None,
                               None, None)
    assert rc == -1 and b"budget" in L.sa_hip_last_error()


def test_loads_next_to_torch_hip_runtime():
    """Inside a torch process the HIP runtime is torch's own libamdhip64; the
    library must not need symbol versions newer than that runtime has."""
    import torch  # noqa: F401  (loads torch's HIP runtime first)
    import solidattention_amd as sa
    C.CDLL(sa.LIB_PATH)


def test_local_causal_argument_checks():
    """Invalid builder arguments are refused before any launch (the
    reference's checks, selection.cpp:18-23, plus the library's limits:
    topk <= 16384, aligned buffers, a large enough workspace).  Any
    head_dim, block size and window pass the checks."""
    import solidattention_amd as sa
    L = sa.lib()
    fake = C.c_void_p(4096)
    assert L.sa_hip_local_causal_workspace_bytes(64, 4, 32) == 64 * 4 * 33 * 4
    # a window past the prompt is the whole prompt: rows of `tokens` floats
    assert L.sa_hip_local_causal_workspace_bytes(64, 4, 1000) == 64 * 4 * 65 * 4
    assert L.sa_hip_local_causal_workspace_bytes(1 << 40, 1 << 30, 1 << 30) == 0  # overflows

    def call(tokens=64, hq=4, hkv=2, d=128, block=32, window=32, topk=4, values=fake, wsb=1 << 30, pq=fake, kv=fake):
        return L.sa_hip_local_causal_representatives(pq, kv, tokens, hq, hkv, d, block, window, topk, values,
                                                     None, None, 0, None, fake, wsb, None)

    bad = [dict(tokens=65), dict(window=0), dict(topk=0), dict(topk=33), dict(hq=3), dict(d=0), dict(block=0),
           dict(block=24), dict(values=None), dict(wsb=16), dict(pq=C.c_void_p(4100)),
           dict(kv=C.c_void_p(4104)), dict(hq=65536 * 2, hkv=65536 * 2, tokens=32),
           dict(tokens=32768, block=32768, topk=16385)]
    for kw in bad:
        assert call(**kw) == -1, kw
        assert L.sa_hip_last_error()


def test_chunked_attention_argument_checks():
    """Chunked attention refuses a non-positive chunk, fewer than two or
    more than 65535 chunks, and a short workspace, before any launch."""
    import solidattention_amd as sa
    L = sa.lib()
    fake = 4096
    kv = sa.PagedKVStruct(fake, fake, fake, fake, fake, fake, 100, 2, 10, 8, 12, 16, 8, 128, 0)
    need = L.sa_hip_attention_workspace_bytes(2, 16, 8, 128, 4)

    def call(chunk=8, chunks=4, wsb=need, sel_stride=10):
        return L.sa_hip_sparse_decode_attention_chunked(C.byref(kv), C.c_void_p(fake), C.c_void_p(fake),
                                                        C.c_void_p(fake), 8, sel_stride, C.c_float(0.1),
                                                        C.c_void_p(fake), C.c_void_p(fake), wsb, chunk, chunks,
                                                        None, None)

    for kw in [dict(chunk=0), dict(chunk=-3), dict(chunks=1), dict(chunks=65536), dict(wsb=need - 4),
               dict(sel_stride=0)]:
        assert call(**kw) == -1, kw
        assert L.sa_hip_last_error()


def test_split_selection_requires_scores():
    """The split selection refuses a null scores buffer before any launch,
    and prefers itself only when the lists leave compute units idle."""
    import solidattention_amd as sa
    L = sa.lib()
    fake = 4096
    kv = sa.PagedKVStruct(fake, fake, fake, fake, fake, fake, 100, 2, 10, 8, 12, 16, 8, 128, 0)
    params = sa.SelectParamsStruct(8, 8, 1, 2, 8, 0, None)
    rc = L.sa_hip_score_select_split(C.byref(kv), C.c_void_p(fake), C.byref(params), C.c_void_p(fake),
                                     C.c_void_p(fake), None, None, None)
    assert rc == -1 and b"scores" in L.sa_hip_last_error()


def test_producer_argument_checks():
    """The projections refuse shapes that are not multiples of 64, short or
    null workspaces and a RoPE theta <= 1 before any launch."""
    import solidattention_amd as sa
    L = sa.lib()
    f = C.c_void_p(4096)
    need = L.sa_hip_linear_workspace_bytes(4, 1024, 2048)
    # the K-slice partial tiles: 64-row tiles, 64 columns x 256 k when that
    # gives the 256 compute units (off the GPU) a workgroup each, else 32
    assert need == 4 * 64 * 2048 * 4  # 1024 -> 2048: 32 x 4 workgroups of 64 columns -> 32 columns
    assert L.sa_hip_linear_workspace_bytes(64, 2048, 1024) == 8 * 64 * 1024 * 4
    assert L.sa_hip_linear(f, f, None, f, 4, 1000, 2048, f, need, None) == -1
    assert L.sa_hip_linear(f, f, None, f, 4, 1024, 2000, f, need, None) == -1
    assert L.sa_hip_linear(f, f, None, f, 4, 1024, 2048, f, need - 4, None) == -1
    assert L.sa_hip_linear(f, f, None, f, 4, 1024, 2048, None, need, None) == -1
    assert L.sa_hip_linear(f, f, None, f, 0, 1024, 2048, f, need, None) == -1
    qn = L.sa_hip_qkv_workspace_bytes(4, 1024, 16, 8)
    # 8 slices of 128 k (two 64-column workgroups per compute unit) of partial
    # tiles + sums of squares
    assert qn == 8 * 64 * 4096 * 4 + 8 * 64 * 4
    args = [f, f, f, f, f, f, f, 4, 1024, 16, 8]
    assert L.sa_hip_qkv_project(*args, C.c_float(1.0), C.c_float(1e-6), f, f, f, f, qn, None) == -1
    assert b"theta" in L.sa_hip_last_error()
    assert L.sa_hip_qkv_project(*args, C.c_float(1e6), C.c_float(1e-6), f, f, f, f, qn - 4, None) == -1
    # q and k are written with 16-byte stores: an unaligned one is refused
    odd = C.c_void_p(4100)
    assert L.sa_hip_qkv_project(*args, C.c_float(1e6), C.c_float(1e-6), odd, f, f, f, qn, None) == -1
    assert L.sa_hip_qkv_project(*args, C.c_float(1e6), C.c_float(1e-6), f, odd, f, f, qn, None) == -1
    assert b"aligned" in L.sa_hip_last_error()
    assert L.sa_hip_rms_norm(f, f, f, 4, 1022, C.c_float(1e-6), None) == -1


def test_noalloc_decode_step_refuses_records_beyond_scratch():
    """The allocation-free decode step refuses split records larger than its
    static scratch before touching the device (safe without a GPU)."""
    import solidattention_amd as sa
    L = sa.lib()
    fake = 4096
    kv = sa.PagedKVStruct(fake, fake, fake, fake, fake, fake, 100, 64, 10, 8, 12, 16, 8, 128, 0)
    params = sa.SelectParamsStruct(8, 8, 1, 2, 8, 0, None)
    records = L.sa_hip_attention_workspace_bytes(64, 16, 8, 128, 64)
    assert records > sa.NOALLOC_SCRATCH_BYTES - sa.NOALLOC_COUNTER_BYTES
    f = C.c_void_p(fake)
    rc = L.sa_hip_decode_step_noalloc(C.byref(kv), f, f, 0, f, C.byref(params), C.c_float(0.1), f, f, f, 64, None,
                                      None)
    assert rc == -1 and b"static scratch" in L.sa_hip_last_error()
    kv.batch = 0
    assert L.sa_hip_decode_step_noalloc(C.byref(kv), f, f, 0, f, C.byref(params), C.c_float(0.1), f, f, f, 1, None,
                                        None) == -1


def test_decode_step_qkv_argument_checks():
    """The producer-fed decode step refuses a null producer, the producer's
    own bad arguments and a head_dim other than 128 before any launch."""
    import solidattention_amd as sa
    L = sa.lib()
    fake = 4096
    f = C.c_void_p(fake)
    kv = sa.PagedKVStruct(fake, fake, fake, fake, fake, fake, 1000, 4, 64, 8, 64, 16, 8, 128, 0)
    params = sa.SelectParamsStruct(8, 8, 1, 2, 8, 0, None)
    ws = L.sa_hip_decode_step_workspace_bytes(C.byref(kv), 1)
    qn = L.sa_hip_qkv_workspace_bytes(4, 1024, 16, 8)
    pr = sa.QkvProducerStruct(fake, fake, 1e-6, fake, fake, fake, fake, fake, fake, 1024, 1e6, 1e-6, fake, fake, fake,
                              fake, qn)

    def call(producer, kvs=kv, nbytes=ws):
        return L.sa_hip_decode_step_qkv(C.byref(kvs), producer, 0, C.byref(params), C.c_float(0.1), f, f, f, f,
                                        nbytes, 1, None, None)

    assert call(None) == -1 and b"null producer" in L.sa_hip_last_error()
    pr.theta = 1.0
    assert call(C.byref(pr)) == -1 and b"theta" in L.sa_hip_last_error()
    pr.theta = 1e6
    pr.workspace_bytes = qn - 4
    assert call(C.byref(pr)) == -1 and b"workspace" in L.sa_hip_last_error()
    pr.workspace_bytes = qn
    pr.hidden = 1000
    assert call(C.byref(pr)) == -1
    pr.hidden = 1024
    assert call(C.byref(pr), nbytes=ws - 4) == -1 and b"workspace" in L.sa_hip_last_error()
    kv64 = sa.PagedKVStruct(fake, fake, fake, fake, fake, fake, 1000, 4, 64, 8, 64, 16, 8, 64, 0)
    assert call(C.byref(pr), kvs=kv64, nbytes=L.sa_hip_decode_step_workspace_bytes(C.byref(kv64), 1)) == -1
    assert b"head_dim 128" in L.sa_hip_last_error()
