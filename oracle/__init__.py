"""ctypes view of the CPU oracle (oracle/liboracle.so) and of the reference
build (oracle/_ref/libsa_ref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg as the checker.  The product path never imports
this package.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libsa_ref.so")
REFERENCE_DIR = "/root/reference"

_SZ = C.c_size_t
_P = C.c_void_p


def build(reference: bool = True) -> None:
    """Compile liboracle.so; also the reference build when its sources exist."""
    subprocess.run(["make", "-s", "-B", "-C", HERE, "liboracle.so"], check=True)
    if reference and os.path.isdir(os.path.join(REFERENCE_DIR, "cpp", "src")):
        subprocess.run(["make", "-s", "-B", "-C", HERE, "ref"], check=True)


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(_P)


class _Lib:
    def __init__(self, path: str):
        self.lib = C.CDLL(path)


_oracle: C.CDLL | None = None
_ref: C.CDLL | None = None


def lib() -> C.CDLL:
    global _oracle
    if _oracle is None:
        if not os.path.exists(LIB_PATH):
            build(reference=False)
        L = C.CDLL(LIB_PATH)
        L.sao_float_to_half.restype = C.c_uint16
        L.sao_float_to_half.argtypes = [C.c_float]
        L.sao_float_to_half_rne.restype = C.c_uint16
        L.sao_float_to_half_rne.argtypes = [C.c_float]
        L.sao_half_to_float.restype = C.c_float
        L.sao_half_to_float.argtypes = [C.c_uint16]
        L.sao_attention_reference.argtypes = [_P, _P, _SZ, _SZ, _SZ, _SZ, C.c_float, _P]
        L.sao_build_local_causal_representatives.argtypes = [_P, _P, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, _P, _P]
        L.sao_build_local_causal_representatives_restated.argtypes = [_P, _P, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, _P, _P,
                                                                 _P]
        L.sao_expf_glibc.restype = C.c_float
        L.sao_expf_glibc.argtypes = [C.c_float]
        L.sao_expf_glibc_table.argtypes = [_P]
        L.sao_expf_glibc_mismatches.restype = C.c_longlong
        L.sao_expf_glibc_mismatches.argtypes = [C.c_uint32, C.c_uint32, C.c_uint32]
        L.sao_mean_key_representatives.argtypes = [_P, _SZ, _SZ, _SZ, _SZ, _P]
        L.sao_select_shared_blocks.argtypes = [_P, _P, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, _P, _P, _P]
        L.sao_paged_score_select.argtypes = [_P, _P, _P, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, _P, _P, _SZ, _P]
        L.sao_paged_sparse_attention.argtypes = [_P, _SZ, _P, _SZ, _P, _P, _P, _P, _SZ, _SZ, _P, _SZ, _SZ, _SZ, _SZ, C.c_float, _P]
        L.sao_paged_append.argtypes = [_P, _SZ, _P, _SZ, _P, _P, _P, _P, _P, _SZ, _SZ, _SZ]
        L.sao_paged_seal.argtypes = [_P, _SZ, _P, _SZ, _P, _P, _P, _P, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ]
        L.sao_pack_blocks.argtypes = [_P, _SZ, _P, _SZ, _P]
        L.sao_run_synthetic_lifecycle.argtypes = [_SZ, _SZ, _P]
        L.sao_topk_argmax.argtypes = [_P, _SZ, _SZ, _P]
        L.sao_compare_prediction.argtypes = [_P, _P, _SZ, _P, _P, _P, _P]
        L.sao_oracle_blocks.argtypes = [_SZ, _SZ, _P]
        L.sao_valid_ticket.argtypes = [_SZ, _SZ, _SZ, _P, _SZ, _SZ, _SZ, _P]
        L.sao_fixture_c1.argtypes = [_SZ, _SZ, _SZ, _SZ, _P, _P]
        L.sao_fixture_c2.argtypes = [_SZ, _SZ, _SZ, _SZ, _P, _P]
        L.sao_p1_query_position.restype = _SZ
        L.sao_p1_query_position.argtypes = [_SZ, _SZ, _SZ]
        L.sao_p1_dense_audit.argtypes = [_P, _P, _P, _SZ, _SZ, _P, _P]
        L.sao_mix64.restype = C.c_uint64
        L.sao_mix64.argtypes = [C.c_uint64]
        L.sao_synth_normal.restype = C.c_float
        L.sao_synth_normal.argtypes = [C.c_uint64, C.c_uint64]
        L.sao_synth_fill_half.argtypes = [C.c_uint64, C.c_uint64, _SZ, _P]
        L.sao_synth_fill_float.argtypes = [C.c_uint64, C.c_uint64, _SZ, _P]
        L.sao_rms_norm.argtypes = [_P, _P, _P, _SZ, _SZ, C.c_float]
        L.sao_linear.argtypes = [_P, _P, _P, _P, _SZ, _SZ, _SZ]
        L.sao_rope_inv_freq.argtypes = [C.c_float, _SZ, _P]
        L.sao_qk_norm_rope.argtypes = [_P, _P, _P, _SZ, _SZ, _SZ, C.c_float, C.c_float]
        _oracle = L
    return _oracle


def ref_available() -> bool:
    return os.path.exists(REF_PATH)


def ref() -> C.CDLL:
    """The reference's own functions (built from its sources) — a checker of
    the oracle, available only where the reference checkout was present at
    build time."""
    global _ref
    if _ref is None:
        L = C.CDLL(REF_PATH)
        L.saref_float_to_half.restype = C.c_uint16
        L.saref_float_to_half.argtypes = [C.c_float]
        L.saref_half_to_float.restype = C.c_float
        L.saref_half_to_float.argtypes = [C.c_uint16]
        L.saref_attention_reference.argtypes = [_P, _P, _SZ, _SZ, _SZ, _SZ, C.c_float, _P]
        L.saref_build_local_causal_representatives.argtypes = [_P, _P, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, _P, _P]
        L.saref_select_shared_blocks.argtypes = [_P, _P, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, _P, _P, _P]
        _ref = L
    return _ref


# --------------------------------------------------------------------------
# numpy-level helpers
# --------------------------------------------------------------------------

def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def attention_reference(kv, query, tokens, hq, hkv, d, scale, use_ref=False):
    kv = _c(kv, np.uint16)
    query = _c(query, np.float32)
    out = np.zeros(hq * d, np.float32)
    f = ref().saref_attention_reference if use_ref else lib().sao_attention_reference
    st = f(_ptr(kv), _ptr(query), tokens, hq, hkv, d, C.c_float(scale), _ptr(out))
    if st != 0:
        raise ValueError("invalid GQA attention dimensions")
    return out.reshape(hq, d)


def local_causal_representatives(prompt_queries, kv, tokens, hq, hkv, d, block, window, topk, use_ref=False):
    prompt_queries = _c(prompt_queries, np.float32)
    kv = _c(kv, np.uint16)
    blocks = tokens // block
    values = np.zeros(hq * blocks * d, np.float32)
    offsets = np.zeros(hq * blocks * topk, np.uint64)
    f = (ref().saref_build_local_causal_representatives if use_ref
         else lib().sao_build_local_causal_representatives)
    st = f(_ptr(prompt_queries), _ptr(kv), tokens, hq, hkv, d, block, window, topk, _ptr(values), _ptr(offsets))
    if st != 0:
        raise ValueError("invalid local-causal representative dimensions")
    return values.reshape(hq, blocks, d), offsets.reshape(hq, blocks, topk)


def local_causal_representatives_restated(prompt_queries, kv, tokens, hq, hkv, d, block, window, topk):
    """The builder with the restated glibc expf (sao_expf_glibc) in place of
    libm's (the GPU builder's arithmetic); returns (values [hq][blocks][d], offsets [hq][blocks][topk],
    received [hq][tokens])."""
    prompt_queries = _c(prompt_queries, np.float32)
    kv = _c(kv, np.uint16)
    blocks = tokens // block
    values = np.zeros(hq * blocks * d, np.float32)
    offsets = np.zeros(hq * blocks * topk, np.uint64)
    received = np.zeros(hq * tokens, np.float32)
    st = lib().sao_build_local_causal_representatives_restated(_ptr(prompt_queries), _ptr(kv), tokens, hq, hkv, d, block,
                                                         window, topk, _ptr(values), _ptr(offsets), _ptr(received))
    if st != 0:
        raise ValueError("invalid local-causal representative dimensions")
    return values.reshape(hq, blocks, d), offsets.reshape(hq, blocks, topk), received.reshape(hq, tokens)


def expf_glibc(x):
    """sao_expf_glibc elementwise over a float32 array."""
    f = lib().sao_expf_glibc
    x = np.asarray(x, np.float32).ravel()
    return np.array([f(float(v)) for v in x], np.float32)


def expf_glibc_table():
    out = np.zeros(32, np.uint64)
    lib().sao_expf_glibc_table(_ptr(out))
    return [int(v) for v in out]


def expf_glibc_mismatches(first_bits, last_bits, stride=1):
    """Floats (bit patterns first, first + stride, ... <= last) where the
    restated expf differs from libm's."""
    return int(lib().sao_expf_glibc_mismatches(first_bits, last_bits, stride))


def mean_key_representatives(kv, tokens, hkv, d, block):
    kv = _c(kv, np.uint16)
    values = np.zeros(hkv * (tokens // block) * d, np.float32)
    st = lib().sao_mean_key_representatives(_ptr(kv), tokens, hkv, d, block, _ptr(values))
    if st != 0:
        raise ValueError("invalid representative dimensions")
    return values.reshape(hkv, tokens // block, d)


def select_shared_blocks(query, reps, heads, blocks, d, budget, init, local, use_ref=False):
    query = _c(query, np.float32)
    reps = _c(reps, np.float32)
    ids = np.zeros(max(blocks, 1), np.uint64)
    count = np.zeros(1, np.uint64)
    scores = np.zeros(max(blocks, 1), np.float32)
    f = ref().saref_select_shared_blocks if use_ref else lib().sao_select_shared_blocks
    st = f(_ptr(query), _ptr(reps), heads, blocks, d, budget, init, local, _ptr(ids), _ptr(count), _ptr(scores))
    if st != 0:
        raise ValueError("invalid representative selection dimensions")
    return ids[: int(count[0])].astype(np.int64), scores[:blocks]


def float_to_half_rne(x):
    x = _c(x, np.float32).ravel()
    f = lib().sao_float_to_half_rne
    return np.array([f(float(v)) for v in x], np.uint16)


def synth_half(seed, first, count):
    out = np.empty(count, np.uint16)
    lib().sao_synth_fill_half(seed, first, count, _ptr(out))
    return out


def synth_float(seed, first, count):
    out = np.empty(count, np.float32)
    lib().sao_synth_fill_float(seed, first, count, _ptr(out))
    return out


def fixture_c1(tokens=128, hq=16, hkv=8, d=128):
    kv = np.zeros(tokens * 2 * hkv * d, np.uint16)
    q = np.zeros(hq * d, np.float32)
    lib().sao_fixture_c1(tokens, hq, hkv, d, _ptr(kv), _ptr(q))
    return kv, q


def fixture_c2(tokens=512, hq=16, hkv=8, d=128):
    kv = np.zeros(tokens * 2 * hkv * d, np.uint16)
    pq = np.zeros(hq * tokens * d, np.float32)
    lib().sao_fixture_c2(tokens, hq, hkv, d, _ptr(kv), _ptr(pq))
    return kv, pq


def paged_score_select(query, reps, sealed, batch, hq, hkv, d, rep_heads, rep_stride,
                       select_groups, budget, init, local, sel_stride=None, want_scores=False):
    sel_stride = sel_stride or budget
    query = _c(query, np.float32)
    reps = _c(reps, np.float32)
    sealed = _c(sealed, np.int32)
    selected = np.full(batch * select_groups * sel_stride, -1, np.int32)
    counts = np.zeros(batch * select_groups, np.int32)
    scores = np.zeros(batch * select_groups * max(rep_stride, 1), np.float32) if want_scores else None
    st = lib().sao_paged_score_select(_ptr(query), _ptr(reps), _ptr(sealed), batch, hq, hkv, d, rep_heads,
                                      rep_stride, select_groups, budget, init, local, _ptr(selected),
                                      _ptr(counts), sel_stride, _ptr(scores))
    if st != 0:
        raise ValueError("invalid paged selection arguments")
    selected = selected.reshape(batch, select_groups, sel_stride)
    counts = counts.reshape(batch, select_groups)
    if want_scores:
        return selected, counts, scores.reshape(batch, select_groups, rep_stride)
    return selected, counts


def paged_sparse_attention(pool, page_tokens, block_table, seq_len, sealed, selected, counts,
                           select_groups, query, batch, hq, hkv, d, scale):
    pool = _c(pool, np.uint16)
    block_table = _c(block_table, np.int32)
    seq_len = _c(seq_len, np.int32)
    sealed = _c(sealed, np.int32)
    selected = _c(selected, np.int32)
    counts = _c(counts, np.int32)
    query = _c(query, np.float32)
    sel_stride = selected.shape[-1]
    table_stride = block_table.shape[-1]
    out = np.zeros(batch * hq * d, np.float32)
    st = lib().sao_paged_sparse_attention(_ptr(pool), page_tokens, _ptr(block_table), table_stride,
                                          _ptr(seq_len), _ptr(sealed), _ptr(selected), _ptr(counts),
                                          sel_stride, select_groups, _ptr(query), batch, hq, hkv, d,
                                          C.c_float(scale), _ptr(out))
    if st != 0:
        raise ValueError("invalid paged attention arguments")
    return out.reshape(batch, hq, d)


def paged_append(pool, page_tokens, block_table, seq_len, k=None, v=None, k16=None, v16=None,
                 batch=None, hkv=None, d=None):
    """In-place on pool (uint16 array) and seq_len (int32 array)."""
    block_table = _c(block_table, np.int32)
    assert pool.dtype == np.uint16 and pool.flags.c_contiguous
    assert seq_len.dtype == np.int32 and seq_len.flags.c_contiguous
    k = None if k is None else _c(k, np.float32)
    v = None if v is None else _c(v, np.float32)
    k16 = None if k16 is None else _c(k16, np.uint16)
    v16 = None if v16 is None else _c(v16, np.uint16)
    st = lib().sao_paged_append(_ptr(pool), page_tokens, _ptr(block_table), block_table.shape[-1],
                                _ptr(seq_len), _ptr(k), _ptr(v), _ptr(k16), _ptr(v16), batch, hkv, d)
    if st != 0:
        raise ValueError("invalid append arguments")


def paged_seal(pool, page_tokens, block_table, seq_len, sealed, generation, reps, rep_heads,
               rep_stride, batch, hq, hkv, d, local_tokens):
    """In-place on sealed, generation and reps."""
    block_table = _c(block_table, np.int32)
    seq_len = _c(seq_len, np.int32)
    for a in (sealed, generation):
        assert a.dtype == np.int32 and a.flags.c_contiguous
    assert reps.dtype == np.float32 and reps.flags.c_contiguous
    st = lib().sao_paged_seal(_ptr(_c(pool, np.uint16)), page_tokens, _ptr(block_table),
                              block_table.shape[-1], _ptr(seq_len), _ptr(sealed), _ptr(generation),
                              _ptr(reps), rep_heads, rep_stride, batch, hq, hkv, d, local_tokens)
    if st != 0:
        raise ValueError("invalid seal arguments")


class LifecycleResult(C.Structure):
    _fields_ = [("sealed_blocks", _SZ), ("representative_head_audits", _SZ),
                ("resident_tail_tokens", _SZ), ("generation", _SZ), ("store_bytes", _SZ),
                ("sealed_bytes_fnv", C.c_uint64)]


def run_synthetic_lifecycle(layers=28, decode_tokens=512):
    r = LifecycleResult()
    st = lib().sao_run_synthetic_lifecycle(layers, decode_tokens, C.byref(r))
    return st, r


def compare_prediction(predicted, oracle_set):
    n = len(predicted)
    p = np.array(predicted, np.uint64)
    o = np.array(oracle_set, np.uint64)
    hits = np.zeros(1, np.uint64)
    misses = np.zeros(max(n, 1), np.uint64)
    slots = np.zeros(max(n, 1), np.uint64)
    mc = np.zeros(1, np.uint64)
    st = lib().sao_compare_prediction(_ptr(p), _ptr(o), n, _ptr(hits), _ptr(misses), _ptr(slots), _ptr(mc))
    m = int(mc[0])
    return st, int(hits[0]), misses[:m].astype(np.int64).tolist(), slots[:m].astype(np.int64).tolist()


def oracle_blocks(step, layer):
    out = np.zeros(4, np.uint64)
    lib().sao_oracle_blocks(step, layer, _ptr(out))
    return out.astype(np.int64).tolist()


def p1_dense_audit(kv, prompt_queries, reps, steps, layers):
    mass = np.zeros(1, np.float64)
    recall = np.zeros(1, np.float64)
    st = lib().sao_p1_dense_audit(_ptr(_c(kv, np.uint16)), _ptr(_c(prompt_queries, np.float32)),
                                  _ptr(_c(reps, np.float32)), steps, layers, _ptr(mass), _ptr(recall))
    if st != 0:
        raise ValueError("dense audit failed")
    return float(mass[0]), float(recall[0])


# --------------------------------------------------------------------------
# query producer / output consumer (qwen_layer_main.cpp:125-183)
# --------------------------------------------------------------------------

def rms_norm(x, w, eps=1e-6):
    x = _c(x, np.float32)
    w = _c(w, np.float32)
    rows, width = x.shape
    out = np.zeros_like(x)
    if lib().sao_rms_norm(_ptr(x), _ptr(w), _ptr(out), rows, width, C.c_float(eps)) != 0:
        raise ValueError("invalid rms_norm arguments")
    return out


def linear(x, w, residual=None):
    """y = x @ w.T (+ residual); w is [out][in] as the reference stores it."""
    x = _c(x, np.float32)
    w = _c(w, np.float32)
    rows, n_in = x.shape
    n_out = w.shape[0]
    y = np.zeros((rows, n_out), np.float32)
    res = None if residual is None else _c(residual, np.float32)
    if lib().sao_linear(_ptr(x), _ptr(w), _ptr(res), _ptr(y), rows, n_in, n_out) != 0:
        raise ValueError("invalid linear arguments")
    return y


def rope_inv_freq(theta, head_dim):
    f = np.zeros(head_dim // 2, np.float32)
    lib().sao_rope_inv_freq(C.c_float(theta), head_dim, _ptr(f))
    return f


def qk_norm_rope(x, w, positions, theta=1e6, eps=1e-6):
    """x [rows][heads][head_dim] -> new array: head RMS norm with w (None:
    none), then RoPE at positions [rows] (None: none)."""
    x = np.array(x, dtype=np.float32, copy=True, order="C")
    rows, heads, hd = x.shape
    wv = None if w is None else _c(w, np.float32)
    pos = None if positions is None else _c(positions, np.int32)
    if lib().sao_qk_norm_rope(_ptr(x), _ptr(wv), _ptr(pos), rows, heads, hd, C.c_float(theta),
                              C.c_float(eps)) != 0:
        raise ValueError("invalid qk_norm_rope arguments")
    return x
