"""Python binding of the MI355X KV-cache decode hot path (libsa_hip.so).

ctypes over the C-ABI of include/sa_hip.h.  Device memory and streams come
from PyTorch (plumbing only); every computation runs in the HIP library.
There is no CPU fallback: loading fails loudly when libsa_hip.so is missing.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.dirname(PKG_DIR)
LIB_PATH = os.path.join(LIB_DIR, "libsa_hip.so")

PAGE_TOKENS = 32
HEAD_DIM = 128

STATUS_BAD_PAGE = 1
STATUS_BAD_BLOCK = 2
STATUS_BAD_LENGTH = 4
STATUS_CAPACITY = 8
STATUS_BAD_BUDGET = 16


class SaHipError(RuntimeError):
    pass


class PagedKVStruct(C.Structure):
    """Mirror of sa_paged_kv (include/sa_hip.h)."""
    _fields_ = [
        ("pool", C.c_void_p), ("block_table", C.c_void_p), ("seq_len", C.c_void_p),
        ("sealed", C.c_void_p), ("generation", C.c_void_p), ("reps", C.c_void_p),
        ("num_pages", C.c_int64), ("batch", C.c_int32), ("table_stride", C.c_int32),
        ("rep_heads", C.c_int32), ("rep_stride", C.c_int32), ("query_heads", C.c_int32),
        ("kv_heads", C.c_int32), ("head_dim", C.c_int32), ("reserved", C.c_int32),
    ]


class SelectParamsStruct(C.Structure):
    """Mirror of sa_select_params (include/sa_hip.h)."""
    _fields_ = [("select_groups", C.c_int32), ("budget_blocks", C.c_int32),
                ("init_blocks", C.c_int32), ("local_blocks", C.c_int32),
                ("sel_stride", C.c_int32), ("reserved", C.c_int32), ("budgets", C.c_void_p)]


class OnlineSealStruct(C.Structure):
    """Mirror of sa_online_seal (include/sa_hip.h)."""
    _fields_ = [("query_ring", C.c_void_p), ("ring_tokens", C.c_int32), ("local_window", C.c_int32),
                ("topk", C.c_int32), ("reserved", C.c_int32)]


class QkvProducerStruct(C.Structure):
    """Mirror of sa_qkv_producer (include/sa_hip.h)."""
    _fields_ = [("hidden_rows", C.c_void_p), ("input_norm", C.c_void_p), ("input_eps", C.c_float),
                ("wq", C.c_void_p), ("wk", C.c_void_p), ("wv", C.c_void_p), ("q_norm", C.c_void_p),
                ("k_norm", C.c_void_p), ("positions", C.c_void_p), ("hidden", C.c_int32), ("theta", C.c_float),
                ("eps", C.c_float), ("q", C.c_void_p), ("k", C.c_void_p), ("v", C.c_void_p),
                ("workspace", C.c_void_p), ("workspace_bytes", C.c_size_t)]


# name -> (restype, argtypes)
_P, _I32, _I64, _SZ, _F = C.c_void_p, C.c_int32, C.c_int64, C.c_size_t, C.c_float
_KV = C.POINTER(PagedKVStruct)
EXPORTS = {
    "sa_hip_last_error": (C.c_char_p, []),
    "sa_hip_abi_version": (C.c_int, []),
    "sa_hip_device_count": (C.c_int, []),
    "sa_hip_attention_workspace_bytes": (_SZ, [_I32, _I32, _I32, _I32, _I32]),
    "sa_hip_attention_default_splits": (_I32, [_I32, _I32, _I32]),
    "sa_hip_attention_splits_for": (_I32, [_I32, _I32, _I32, _I32]),
    "sa_hip_sparse_decode_attention": (C.c_int, [_KV, _P, _P, _P, _I32, _I32, _F, _P, _P, _SZ, _I32, _P, _P]),
    "sa_hip_sparse_decode_attention_partial": (C.c_int, [_KV, _P, _P, _P, _I32, _I32, _F, _I32, _P, _SZ, _I32, _I32,
                                                         _I32, _P, _P]),
    "sa_hip_attention_merge": (C.c_int, [_KV, _P, _SZ, _I32, _P, _P]),
    "sa_hip_rms_norm": (C.c_int, [_P, _P, _P, _I32, _I32, _F, _P]),
    "sa_hip_linear_workspace_bytes": (_SZ, [_I32, _I32, _I32]),
    "sa_hip_linear": (C.c_int, [_P, _P, _P, _P, _I32, _I32, _I32, _P, _SZ, _P]),
    "sa_hip_qkv_workspace_bytes": (_SZ, [_I32, _I32, _I32, _I32]),
    "sa_hip_qkv_project": (C.c_int, [_P, _P, _P, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _F, _F, _P, _P, _P, _P,
                                     _SZ, _P]),
    "sa_hip_qkv_project_rms": (C.c_int, [_P, _P, _F, _P, _P, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _F, _F, _P,
                                         _P, _P, _P, _SZ, _P]),
    "sa_store_open": (C.c_void_p, [C.c_char_p, _I64, _I64, _I64, _I32, _I32]),
    "sa_store_close": (None, [_P]),
    "sa_store_is_direct": (C.c_int, [_P]),
    "sa_store_bytes": (_I64, [_P]),
    "sa_store_bounced": (_I64, [_P]),
    "sa_store_submit_reads": (_I64, [_P, _I64, _P, _I32, _P]),
    "sa_store_submit_writes": (_I64, [_P, _I64, _P, _I32, _P]),
    "sa_store_wait": (C.c_int, [_P, _I64]),
    "sa_store_read_blocks": (C.c_int, [_P, _I64, _P, _I32, _P]),
    "sa_store_write_blocks": (C.c_int, [_P, _I64, _P, _I32, _P]),
    "sa_store_sync": (C.c_int, [_P]),
    "sa_store_commit_marker": (C.c_int, [C.c_char_p, C.c_char_p, C.c_char_p]),
    "sa_hip_pages_to_host_async": (C.c_int, [_P, _I64, _I64, _P, _I32, _P, _P, _P, _P]),
    "sa_hip_score_select_split": (C.c_int, [_KV, _P, C.POINTER(SelectParamsStruct), _P, _P, _P, _P, _P]),
    "sa_hip_score_select_split_preferred": (C.c_int, [_KV, C.POINTER(SelectParamsStruct)]),
    "sa_hip_score_select_chunked_workspace_bytes": (_SZ, [_KV, C.POINTER(SelectParamsStruct)]),
    "sa_hip_score_select_chunked": (C.c_int, [_KV, _P, C.POINTER(SelectParamsStruct), _P, _P, _P, _SZ, _P, _P]),
    "sa_hip_attention_chunked_workspace_bytes": (_SZ, [_I32, _I32, _I32, _I32, _I32]),
    "sa_hip_sparse_decode_attention_chunked": (C.c_int, [_KV, _P, _P, _P, _I32, _I32, _F, _P, _P, _SZ, _I32, _I32,
                                                         _P, _P]),
    "sa_hip_contiguous_workspace_bytes": (_SZ, [_I64, _I32, _I32, _I32]),
    "sa_hip_attention_contiguous": (C.c_int, [_P, _P, _I64, _I32, _I32, _I32, _F, _P, _P, _SZ, _P]),
    "sa_hip_consume_checksum": (C.c_int, [_P, _I32, _P, _P]),
    "sa_hip_score_select": (C.c_int, [_KV, _P, C.POINTER(SelectParamsStruct), _P, _P, _P, _P, _P]),
    "sa_hip_select_attend_fused": (C.c_int, [_KV, C.POINTER(SelectParamsStruct), _I32]),
    "sa_hip_select_attend_default_splits": (_I32, [_KV, C.POINTER(SelectParamsStruct)]),
    "sa_hip_select_attend": (C.c_int, [_KV, _P, C.POINTER(SelectParamsStruct), _F, _P, _P, _P, _P, _SZ, _I32, _P,
                                       _P]),
    "sa_hip_decode_step_workspace_bytes": (_SZ, [_KV, _I32]),
    "sa_hip_decode_step": (C.c_int, [_KV, _P, _P, _I32, _P, C.POINTER(SelectParamsStruct), _F, _P, _P, _P, _P, _SZ,
                                     _I32, _P, _P]),
    "sa_hip_decode_step_f16": (C.c_int, [_KV, _P, _P, _I32, _P, C.POINTER(SelectParamsStruct), _F, _P, _P, _P, _P,
                                         _SZ, _I32, _P, _P]),
    "sa_hip_append_seal_online": (C.c_int, [_KV, _P, _P, _I32, _P, C.POINTER(OnlineSealStruct), _P, _P]),
    "sa_hip_decode_step_online": (C.c_int, [_KV, _P, _P, _I32, _P, C.POINTER(OnlineSealStruct),
                                            C.POINTER(SelectParamsStruct), _F, _P, _P, _P, _P, _SZ, _I32, _P, _P]),
    "sa_hip_decode_step_noalloc": (C.c_int, [_KV, _P, _P, _I32, _P, C.POINTER(SelectParamsStruct), _F, _P, _P, _P,
                                             _I32, _P, _P]),
    "sa_hip_decode_step_qkv": (C.c_int, [_KV, C.POINTER(QkvProducerStruct), _I32, C.POINTER(SelectParamsStruct), _F,
                                         _P, _P, _P, _P, _SZ, _I32, _P, _P]),
    "sa_hip_append_seal": (C.c_int, [_KV, _P, _P, _I32, _P, _P]),
    "sa_hip_append_seal_f16": (C.c_int, [_KV, _P, _P, _I32, _P, _P]),
    "sa_hip_seal": (C.c_int, [_KV, _I32, _P, _P]),
    "sa_hip_gather_pages": (C.c_int, [_P, _I64, _I64, _P, _I32, _P, _P, _P]),
    "sa_hip_read_step_bytes": (C.c_int, [_KV, _P, _P, _I32, _I32, _P, _P, _P]),
    "sa_hip_local_causal_workspace_bytes": (_SZ, [_I64, _I32, _I32]),
    "sa_hip_local_causal_representatives": (C.c_int, [_P, _P, _I64, _I32, _I32, _I32, _I32, _I32, _I32, _P, _P, _P,
                                                      _I32, _P, _P, _SZ, _P]),
    "sa_hip_compare_prediction": (C.c_int, [_P, _P, _I32, _P, _P, _P, _P]),
    "sa_hip_fill_pages_async": (C.c_int, [_P, _I64, _P, _P, _P, _I32, _P, _P]),
    "sa_hip_fill_pages_gather_async": (C.c_int, [_P, _I64, _I64, _P, _P, _I64, _P, _I32, _P, _P, _P]),
    "sa_hip_stream_wait_event": (C.c_int, [_P, _P]),
    "sa_hip_fill_synthetic_f16": (C.c_int, [_P, _I64, C.c_uint64, C.c_uint64, _P]),
    "sa_hip_fill_synthetic_f32": (C.c_int, [_P, _I64, C.c_uint64, C.c_uint64, _P]),
}

_lib: C.CDLL | None = None


def build() -> None:
    """Compile libsa_hip.so for gfx950 (hipcc cross-compiles without a GPU)."""
    subprocess.run(["make", "-s", "-B", "-j8", "-C", LIB_DIR], check=True)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise SaHipError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                             "(there is no CPU fallback)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in EXPORTS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(rc: int, what: str = "sa_hip") -> None:
    if rc != 0:
        msg = lib().sa_hip_last_error().decode(errors="replace")
        raise SaHipError(f"{what} failed ({rc}): {msg}")


# --------------------------------------------------------------------------
# torch plumbing helpers (imported lazily so the CPU tests need no GPU)
# --------------------------------------------------------------------------

def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _stream(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)


REP_ROW_FLOATS = 32


def default_rep_stride(blocks):
    """Representative row stride for `blocks` blocks: a multiple of 32 floats,
    so that each head_dim row of [rep head][d][block] starts on a 128-byte
    line and a row of n blocks is fetched as ceil(4 n / 128) lines instead of
    one line more (the scoring kernels read every row with streaming loads,
    so a line shared by two rows is fetched twice)."""
    return (max(int(blocks), 1) + REP_ROW_FLOATS - 1) // REP_ROW_FLOATS * REP_ROW_FLOATS


class PagedKV:
    """Device-resident paged FP16 KV slot pool of one layer.

    pool         uint16 [num_pages, 32, 2, kv_heads, head_dim]
    block_table  int32  [batch, table_stride]
    seq_len      int32  [batch]
    sealed       int32  [batch]
    generation   int32  [batch]
    reps         fp32   [batch, rep_heads, head_dim, rep_stride]
    """

    def __init__(self, batch, query_heads, kv_heads, table_stride, num_pages=None,
                 rep_heads=None, rep_stride=None, head_dim=HEAD_DIM, device="cuda", pool=None):
        import torch
        self.batch, self.query_heads, self.kv_heads = batch, query_heads, kv_heads
        self.head_dim = head_dim
        self.table_stride = table_stride
        self.num_pages = num_pages if num_pages is not None else batch * table_stride
        self.rep_heads = rep_heads if rep_heads is not None else kv_heads
        # a multiple of 32 floats starts every representative row on a
        # 128-byte line (and lets the scoring kernel load 4 blocks per lane)
        self.rep_stride = rep_stride if rep_stride is not None else default_rep_stride(table_stride)
        dev = torch.device(device)
        if pool is None:
            pool = torch.zeros((self.num_pages, PAGE_TOKENS, 2, kv_heads, head_dim),
                               dtype=torch.int16, device=dev).view(torch.uint16)
        self.pool = pool
        self.block_table = torch.zeros((batch, table_stride), dtype=torch.int32, device=dev)
        self.seq_len = torch.zeros(batch, dtype=torch.int32, device=dev)
        self.sealed = torch.zeros(batch, dtype=torch.int32, device=dev)
        self.generation = torch.zeros(batch, dtype=torch.int32, device=dev)
        self.reps = torch.zeros((batch, self.rep_heads, head_dim, self.rep_stride),
                                dtype=torch.float32, device=dev)

    def struct(self) -> PagedKVStruct:
        return PagedKVStruct(
            self.pool.data_ptr(), self.block_table.data_ptr(), self.seq_len.data_ptr(),
            self.sealed.data_ptr(), self.generation.data_ptr(), self.reps.data_ptr(),
            self.num_pages, self.batch, self.table_stride, self.rep_heads, self.rep_stride,
            self.query_heads, self.kv_heads, self.head_dim, 0)

    @property
    def page_bytes(self) -> int:
        return PAGE_TOKENS * 2 * self.kv_heads * self.head_dim * 2

    def sequences(self, first, stop):
        """A view of sequences [first, stop): the same page pool, the rows of
        the tables, lengths, counters and representatives of those sequences
        (no copy).  Calls on disjoint views touch disjoint state, so they may
        run concurrently on different streams (micro-batches)."""
        import copy
        if not 0 <= first < stop <= self.batch:
            raise ValueError(f"sequences [{first}, {stop}) outside the batch of {self.batch}")
        v = copy.copy(self)
        v.batch = stop - first
        v.block_table = self.block_table[first:stop]
        v.seq_len = self.seq_len[first:stop]
        v.sealed = self.sealed[first:stop]
        v.generation = self.generation[first:stop]
        v.reps = self.reps[first:stop]
        return v


def score_select(kv: PagedKV, query, select_groups, budget, init, local, selected=None, counts=None,
                 scores=None, status=None, sel_stride=None, stream=None, budgets=None):
    """budgets: optional device int32 [batch] of per-sequence budgets."""
    import torch
    sel_stride = sel_stride or budget
    dev = query.device
    if selected is None:
        selected = torch.full((kv.batch, select_groups, sel_stride), -1, dtype=torch.int32, device=dev)
    if counts is None:
        counts = torch.zeros((kv.batch, select_groups), dtype=torch.int32, device=dev)
    params = SelectParamsStruct(select_groups, budget, init, local, sel_stride, 0,
                                None if budgets is None else budgets.data_ptr())
    s = kv.struct()
    check(lib().sa_hip_score_select(C.byref(s), _ptr(query), C.byref(params), _ptr(selected), _ptr(counts),
                                    _ptr(scores), _ptr(status), _stream(stream)), "score_select")
    return selected, counts


def score_select_split(kv: PagedKV, query, select_groups, budget, init, local, selected=None, counts=None,
                       scores=None, status=None, sel_stride=None, stream=None, budgets=None):
    """score_select with the scoring spread over 256-block workgroups; scores
    ([batch][select_groups][rep_stride] fp32) is written and returned."""
    import torch
    sel_stride = sel_stride or budget
    dev = query.device
    if selected is None:
        selected = torch.full((kv.batch, select_groups, sel_stride), -1, dtype=torch.int32, device=dev)
    if counts is None:
        counts = torch.zeros((kv.batch, select_groups), dtype=torch.int32, device=dev)
    if scores is None:
        scores = torch.zeros((kv.batch, select_groups, kv.rep_stride), dtype=torch.float32, device=dev)
    params = SelectParamsStruct(select_groups, budget, init, local, sel_stride, 0,
                                None if budgets is None else budgets.data_ptr())
    s = kv.struct()
    check(lib().sa_hip_score_select_split(C.byref(s), _ptr(query), C.byref(params), _ptr(selected), _ptr(counts),
                                          _ptr(scores), _ptr(status), _stream(stream)), "score_select_split")
    return selected, counts, scores


def score_select_chunked_workspace(kv: PagedKV, select_groups, budget, init, local, sel_stride=None):
    """A zeroed workspace for score_select_chunked (reusable across calls that
    do not overlap)."""
    import torch
    params = SelectParamsStruct(select_groups, budget, init, local, sel_stride or budget, 0, None)
    s = kv.struct()
    nbytes = int(lib().sa_hip_score_select_chunked_workspace_bytes(C.byref(s), C.byref(params)))
    return torch.zeros(max(nbytes // 4, 1), dtype=torch.int32, device="cuda"), nbytes


def score_select_chunked(kv: PagedKV, query, select_groups, budget, init, local, workspace, selected=None,
                         counts=None, status=None, sel_stride=None, stream=None, budgets=None):
    """score_select as one launch that splits long lists over workgroups of at
    most 1024 or 2048 blocks (workspace from score_select_chunked_workspace)."""
    import torch
    sel_stride = sel_stride or budget
    dev = query.device
    if selected is None:
        selected = torch.full((kv.batch, select_groups, sel_stride), -1, dtype=torch.int32, device=dev)
    if counts is None:
        counts = torch.zeros((kv.batch, select_groups), dtype=torch.int32, device=dev)
    params = SelectParamsStruct(select_groups, budget, init, local, sel_stride, 0,
                                None if budgets is None else budgets.data_ptr())
    s = kv.struct()
    check(lib().sa_hip_score_select_chunked(C.byref(s), _ptr(query), C.byref(params), _ptr(selected),
                                            _ptr(counts), _ptr(workspace), workspace.numel() * workspace.element_size(),
                                            _ptr(status), _stream(stream)), "score_select_chunked")
    return selected, counts


def score_select_split_preferred(kv: PagedKV, select_groups, budget, init, local, sel_stride=None) -> bool:
    params = SelectParamsStruct(select_groups, budget, init, local, sel_stride or budget, 0, None)
    s = kv.struct()
    return bool(lib().sa_hip_score_select_split_preferred(C.byref(s), C.byref(params)))


def rms_norm(x, w, eps=1e-6, out=None, stream=None):
    """x [rows][width] fp32 -> x * rsqrt(mean(x^2) + eps) * w."""
    import torch
    rows, width = x.shape
    if out is None:
        out = torch.empty_like(x)
    check(lib().sa_hip_rms_norm(_ptr(x), _ptr(w), _ptr(out), rows, width, C.c_float(eps), _stream(stream)),
          "rms_norm")
    return out


def linear(x, w, residual=None, out=None, workspace=None, stream=None):
    """y = x @ w.T (+ residual); w is [out][in] fp32."""
    import torch
    rows, n_in = x.shape
    n_out = w.shape[0]
    if out is None:
        out = torch.empty((rows, n_out), dtype=torch.float32, device=x.device)
    nbytes = lib().sa_hip_linear_workspace_bytes(rows, n_in, n_out)
    if workspace is None:  # the K-slice partial tiles (no initialisation needed)
        workspace = torch.empty(max(nbytes // 4, 1), dtype=torch.float32, device=x.device)
    check(lib().sa_hip_linear(_ptr(x), _ptr(w), _ptr(residual), _ptr(out), rows, n_in, n_out, _ptr(workspace),
                              workspace.numel() * 4, _stream(stream)), "linear")
    return out


def qkv_project(x, wq, wk, wv, q_norm, k_norm, positions, q_heads, kv_heads, theta=1e6, eps=1e-6, q=None, k=None,
                v=None, workspace=None, stream=None, input_norm=None, input_eps=1e-6):
    """Normalised hidden x [rows][hidden] -> q [rows][q_heads][128] and
    k [rows][kv_heads][128] (head RMS norm + RoPE at positions [rows]) and
    v [rows][kv_heads][128].  With input_norm, x is the raw hidden and its
    RMSNorm (weight input_norm) runs in the same launch."""
    import torch
    rows, hidden = x.shape
    dev = x.device
    q = q if q is not None else torch.empty((rows, q_heads, HEAD_DIM), dtype=torch.float32, device=dev)
    k = k if k is not None else torch.empty((rows, kv_heads, HEAD_DIM), dtype=torch.float32, device=dev)
    v = v if v is not None else torch.empty((rows, kv_heads, HEAD_DIM), dtype=torch.float32, device=dev)
    nbytes = lib().sa_hip_qkv_workspace_bytes(rows, hidden, q_heads, kv_heads)
    if workspace is None:  # the K-slice partial tiles (no initialisation needed)
        workspace = torch.empty(max(nbytes // 4, 1), dtype=torch.float32, device=dev)
    if input_norm is None:
        check(lib().sa_hip_qkv_project(_ptr(x), _ptr(wq), _ptr(wk), _ptr(wv), _ptr(q_norm), _ptr(k_norm),
                                       _ptr(positions), rows, hidden, q_heads, kv_heads, C.c_float(theta),
                                       C.c_float(eps), _ptr(q), _ptr(k), _ptr(v), _ptr(workspace),
                                       workspace.numel() * 4, _stream(stream)), "qkv_project")
    else:
        check(lib().sa_hip_qkv_project_rms(_ptr(x), _ptr(input_norm), C.c_float(input_eps), _ptr(wq), _ptr(wk),
                                           _ptr(wv), _ptr(q_norm), _ptr(k_norm), _ptr(positions), rows, hidden,
                                           q_heads, kv_heads, C.c_float(theta), C.c_float(eps), _ptr(q), _ptr(k),
                                           _ptr(v), _ptr(workspace), workspace.numel() * 4, _stream(stream)),
              "qkv_project_rms")
    return q, k, v


STORE_CREATE, STORE_DIRECT = 1, 2


class MainStore:
    """The main KV store file (include/sa_store.h): block `block` of layer
    `layer` at byte (layer * blocks_per_layer + block) * block_bytes.
    Buffers are numpy arrays or tensors (pinned host memory for O_DIRECT:
    4096-byte aligned); block ids are int64 sequences."""

    def __init__(self, path, layers, blocks_per_layer, block_bytes, create=False, direct=True, threads=8):
        flags = (STORE_CREATE if create else 0) | (STORE_DIRECT if direct else 0)
        self.layers, self.blocks_per_layer, self.block_bytes = layers, blocks_per_layer, block_bytes
        self.handle = lib().sa_store_open(os.fsencode(path), layers, blocks_per_layer, block_bytes, flags, threads)
        if not self.handle:
            raise SaHipError(f"store_open failed: {lib().sa_hip_last_error().decode(errors='replace')}")

    @property
    def direct(self) -> bool:
        return bool(lib().sa_store_is_direct(self.handle))

    @property
    def nbytes(self) -> int:
        return int(lib().sa_store_bytes(self.handle))

    @property
    def bounced(self) -> int:
        return int(lib().sa_store_bounced(self.handle))

    @staticmethod
    def _ids(blocks):
        import numpy as np
        ids = np.ascontiguousarray(np.asarray(blocks, dtype=np.int64))
        return ids, ids.ctypes.data_as(C.c_void_p)

    @staticmethod
    def _buf(buf):
        return C.c_void_p(buf.data_ptr()) if hasattr(buf, "data_ptr") else buf.ctypes.data_as(C.c_void_p)

    def submit_reads(self, layer, blocks, dst) -> int:
        ids, p = self._ids(blocks)
        bid = lib().sa_store_submit_reads(self.handle, layer, p, ids.size, self._buf(dst))
        if bid < 0:
            check(int(bid), "store_submit_reads")
        return bid

    def submit_writes(self, layer, blocks, src) -> int:
        ids, p = self._ids(blocks)
        bid = lib().sa_store_submit_writes(self.handle, layer, p, ids.size, self._buf(src))
        if bid < 0:
            check(int(bid), "store_submit_writes")
        return bid

    def wait(self, batch) -> None:
        check(lib().sa_store_wait(self.handle, batch), "store_wait")

    def read(self, layer, blocks, dst) -> None:
        ids, p = self._ids(blocks)
        check(lib().sa_store_read_blocks(self.handle, layer, p, ids.size, self._buf(dst)), "store_read_blocks")

    def write(self, layer, blocks, src) -> None:
        ids, p = self._ids(blocks)
        check(lib().sa_store_write_blocks(self.handle, layer, p, ids.size, self._buf(src)), "store_write_blocks")

    def sync(self) -> None:
        check(lib().sa_store_sync(self.handle), "store_sync")

    def close(self) -> None:
        if self.handle:
            lib().sa_store_close(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def commit_marker(directory, name, body) -> None:
    check(lib().sa_store_commit_marker(os.fsencode(directory), name.encode(), body.encode()), "store_commit_marker")


def pages_to_host_async(pool, page_bytes, num_pages, pages, dst, copy_stream, after_event=None, done_event=None):
    """D2H of pool pages `pages` (host int32 sequence) into pinned `dst` on
    copy_stream after after_event; records done_event."""
    import numpy as np
    ids = np.ascontiguousarray(np.asarray(pages, dtype=np.int32))
    ev = lambda e: None if e is None else C.c_void_p(e.cuda_event if hasattr(e, "cuda_event") else e)
    check(lib().sa_hip_pages_to_host_async(_ptr(pool), page_bytes, num_pages, ids.ctypes.data_as(C.c_void_p),
                                           ids.size, C.c_void_p(dst.data_ptr()), _stream(copy_stream),
                                           ev(after_event), ev(done_event)), "pages_to_host_async")


def select_attend(kv: PagedKV, query, select_groups, budget, init, local, scale, selected=None, counts=None,
                  out=None, splits=1, workspace=None, status=None, sel_stride=None, stream=None, budgets=None):
    """score_select followed by sparse_decode_attention; one fused launch when
    select_attend_fused() says so.  Returns (selected, counts, out)."""
    import torch
    sel_stride = sel_stride or budget
    dev = query.device
    if selected is None:
        selected = torch.full((kv.batch, select_groups, sel_stride), -1, dtype=torch.int32, device=dev)
    if counts is None:
        counts = torch.zeros((kv.batch, select_groups), dtype=torch.int32, device=dev)
    if out is None:
        out = torch.empty((kv.batch, kv.query_heads, kv.head_dim), dtype=torch.float32, device=dev)
    nbytes = lib().sa_hip_attention_workspace_bytes(kv.batch, kv.query_heads, kv.kv_heads, kv.head_dim, splits)
    if workspace is None and nbytes:
        workspace = torch.zeros(nbytes // 4, dtype=torch.float32, device=dev)
    params = SelectParamsStruct(select_groups, budget, init, local, sel_stride, 0,
                                None if budgets is None else budgets.data_ptr())
    s = kv.struct()
    check(lib().sa_hip_select_attend(C.byref(s), _ptr(query), C.byref(params), C.c_float(scale), _ptr(selected),
                                     _ptr(counts), _ptr(out), _ptr(workspace) if nbytes else None, nbytes, splits,
                                     _ptr(status), _stream(stream)), "select_attend")
    return selected, counts, out


def decode_step_workspace(kv: PagedKV, splits=1, device="cuda"):
    """Zeroed workspace for decode_step (arrival counters + split records)."""
    import torch
    n = lib().sa_hip_decode_step_workspace_bytes(C.byref(kv.struct()), splits)
    return torch.zeros(max(n // 4, 1), dtype=torch.int32, device=device), n


def decode_step(kv: PagedKV, k, v, local_tokens, query, select_groups, budget, init, local, scale, workspace,
                selected=None, counts=None, out=None, splits=1, status=None, sel_stride=None, stream=None,
                budgets=None):
    """append_seal + score_select + sparse_decode_attention for one layer; one
    fused launch when select_attend_fused() says so.  k, v: fp32 (converted
    round-to-nearest-even) or uint16 FP16 bits, [batch, kv_heads, head_dim].
    workspace: from decode_step_workspace() (kept zeroed between calls).
    Returns (selected, counts, out)."""
    import torch
    sel_stride = sel_stride or budget
    dev = query.device
    if selected is None:
        selected = torch.full((kv.batch, select_groups, sel_stride), -1, dtype=torch.int32, device=dev)
    if counts is None:
        counts = torch.zeros((kv.batch, select_groups), dtype=torch.int32, device=dev)
    if out is None:
        out = torch.empty((kv.batch, kv.query_heads, kv.head_dim), dtype=torch.float32, device=dev)
    params = SelectParamsStruct(select_groups, budget, init, local, sel_stride, 0,
                                None if budgets is None else budgets.data_ptr())
    s = kv.struct()
    nbytes = workspace.numel() * workspace.element_size()
    fn = lib().sa_hip_decode_step_f16 if k.dtype == torch.uint16 else lib().sa_hip_decode_step
    check(fn(C.byref(s), _ptr(k), _ptr(v), local_tokens, _ptr(query), C.byref(params), C.c_float(scale),
             _ptr(selected), _ptr(counts), _ptr(out), _ptr(workspace), nbytes, splits, _ptr(status),
             _stream(stream)), "decode_step")
    return selected, counts, out


def decode_step_qkv(kv: PagedKV, x, wq, wk, wv, q_norm, k_norm, positions, q, k, v, qkv_workspace, local_tokens,
                    select_groups, budget, init, local, scale, workspace, input_norm=None, input_eps=1e-6, theta=1e6,
                    eps=1e-6, selected=None, counts=None, out=None, splits=1, status=None, sel_stride=None,
                    stream=None, budgets=None):
    """qkv_project (x [batch][hidden] -> q, k, v) followed by decode_step(kv,
    k, v, local_tokens, q, ...): two launches where the one-launch step takes
    the producer's epilogue (1-2 query heads per KV head), else the two calls.
    q, k, v are written as qkv_project writes them.  Returns (selected,
    counts, out)."""
    import torch
    sel_stride = sel_stride or budget
    dev = x.device
    if selected is None:
        selected = torch.full((kv.batch, select_groups, sel_stride), -1, dtype=torch.int32, device=dev)
    if counts is None:
        counts = torch.zeros((kv.batch, select_groups), dtype=torch.int32, device=dev)
    if out is None:
        out = torch.empty((kv.batch, kv.query_heads, kv.head_dim), dtype=torch.float32, device=dev)
    params = SelectParamsStruct(select_groups, budget, init, local, sel_stride, 0,
                                None if budgets is None else budgets.data_ptr())
    pr = QkvProducerStruct(x.data_ptr(), None if input_norm is None else input_norm.data_ptr(), input_eps,
                           wq.data_ptr(), wk.data_ptr(), wv.data_ptr(), q_norm.data_ptr(), k_norm.data_ptr(),
                           positions.data_ptr(), x.shape[1], theta, eps, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                           qkv_workspace.data_ptr(), qkv_workspace.numel() * qkv_workspace.element_size())
    s = kv.struct()
    nbytes = workspace.numel() * workspace.element_size()
    check(lib().sa_hip_decode_step_qkv(C.byref(s), C.byref(pr), local_tokens, C.byref(params), C.c_float(scale),
                                       _ptr(selected), _ptr(counts), _ptr(out), _ptr(workspace), nbytes, splits,
                                       _ptr(status), _stream(stream)), "decode_step_qkv")
    return selected, counts, out


class OnlineSeal:
    """The InfLLM online seal's query ring ([batch, query_heads, ring_tokens,
    128] fp32 on the device) and builder parameters (sa_online_seal)."""

    def __init__(self, kv: PagedKV, ring_tokens=PAGE_TOKENS, window=PAGE_TOKENS, topk=4, device="cuda"):
        import torch
        self.ring = torch.zeros((kv.batch, kv.query_heads, ring_tokens, kv.head_dim), dtype=torch.float32,
                                device=device)
        self.ring_tokens, self.window, self.topk = ring_tokens, window, topk

    def struct(self) -> OnlineSealStruct:
        return OnlineSealStruct(self.ring.data_ptr(), self.ring_tokens, self.window, self.topk, 0)


def append_seal_online(kv: PagedKV, k, v, local_tokens, query, seal: OnlineSeal, status=None, stream=None):
    s = kv.struct()
    o = seal.struct()
    check(lib().sa_hip_append_seal_online(C.byref(s), _ptr(k), _ptr(v), local_tokens, _ptr(query), C.byref(o),
                                          _ptr(status), _stream(stream)), "append_seal_online")


def decode_step_online(kv: PagedKV, k, v, local_tokens, query, seal: OnlineSeal, select_groups, budget, init, local,
                       scale, workspace, selected=None, counts=None, out=None, splits=1, status=None,
                       sel_stride=None, stream=None, budgets=None):
    """decode_step (fp32 k/v) with the InfLLM online seal: the step's queries
    go to seal.ring and a sealed block gets the local-causal representative
    of every query head (kv.rep_heads == kv.query_heads)."""
    import torch
    sel_stride = sel_stride or budget
    dev = query.device
    if selected is None:
        selected = torch.full((kv.batch, select_groups, sel_stride), -1, dtype=torch.int32, device=dev)
    if counts is None:
        counts = torch.zeros((kv.batch, select_groups), dtype=torch.int32, device=dev)
    if out is None:
        out = torch.empty((kv.batch, kv.query_heads, kv.head_dim), dtype=torch.float32, device=dev)
    params = SelectParamsStruct(select_groups, budget, init, local, sel_stride, 0,
                                None if budgets is None else budgets.data_ptr())
    s = kv.struct()
    o = seal.struct()
    nbytes = workspace.numel() * workspace.element_size()
    check(lib().sa_hip_decode_step_online(C.byref(s), _ptr(k), _ptr(v), local_tokens, _ptr(query), C.byref(o),
                                          C.byref(params), C.c_float(scale), _ptr(selected), _ptr(counts), _ptr(out),
                                          _ptr(workspace), nbytes, splits, _ptr(status), _stream(stream)),
          "decode_step_online")
    return selected, counts, out


NOALLOC_SCRATCH_BYTES = 4 << 20
NOALLOC_COUNTER_BYTES = 256 << 10


def decode_step_noalloc(kv: PagedKV, k, v, local_tokens, query, select_groups, budget, init, local, scale,
                        selected, counts, out, splits=1, status=None, sel_stride=None, stream=None, budgets=None):
    """decode_step without a workspace: the library's static per-GPU scratch
    (sa_hip_decode_step_noalloc).  fp32 k/v; the caller passes the outputs.
    Calls that overlap on one GPU race."""
    sel_stride = sel_stride or budget
    params = SelectParamsStruct(select_groups, budget, init, local, sel_stride, 0,
                                None if budgets is None else budgets.data_ptr())
    s = kv.struct()
    check(lib().sa_hip_decode_step_noalloc(C.byref(s), _ptr(k), _ptr(v), local_tokens, _ptr(query), C.byref(params),
                                           C.c_float(scale), _ptr(selected), _ptr(counts), _ptr(out), splits,
                                           _ptr(status), _stream(stream)), "decode_step_noalloc")
    return selected, counts, out


def select_attend_default_splits(kv: PagedKV, select_groups, budget) -> int:
    """1 where the fused launch applies and fills the device, else the split
    count of the separate attention launch."""
    params = SelectParamsStruct(select_groups, budget, 0, 0, budget, 0, None)
    return int(lib().sa_hip_select_attend_default_splits(C.byref(kv.struct()), C.byref(params)))


def select_attend_fused(kv: PagedKV, select_groups, splits=1, sel_stride=None, budget=None) -> bool:
    """Whether select_attend / decode_step run as one launch for this
    geometry.  sel_stride: the row stride of the caller's selected[] (the
    fused launch at 4 query heads per KV head keeps up to 2048 ids per list
    on chip); defaults to budget, which defaults to 1."""
    budget = budget or 1
    sel_stride = sel_stride or budget
    params = SelectParamsStruct(select_groups, budget, 0, 0, sel_stride, 0, None)
    s = kv.struct()
    return bool(lib().sa_hip_select_attend_fused(C.byref(s), C.byref(params), splits))


def attention_workspace(kv: PagedKV, splits, device="cuda"):
    import torch
    n = lib().sa_hip_attention_workspace_bytes(kv.batch, kv.query_heads, kv.kv_heads, kv.head_dim, splits)
    return torch.zeros(max(n // 4, 1), dtype=torch.float32, device=device), n


def default_splits(batch, kv_heads, pages_hint, query_heads=None):
    """Split count of the library for a launch; query_heads defaults to two
    per KV head."""
    if query_heads is None:
        return int(lib().sa_hip_attention_default_splits(batch, kv_heads, pages_hint))
    return int(lib().sa_hip_attention_splits_for(batch, query_heads, kv_heads, pages_hint))


def sparse_decode_attention(kv: PagedKV, query, selected, counts, scale, out=None, splits=None,
                            workspace=None, status=None, stream=None):
    import torch
    select_groups, sel_stride = selected.shape[1], selected.shape[2]
    if splits is None:
        splits = default_splits(kv.batch, kv.kv_heads, sel_stride + 2, kv.query_heads)
    if out is None:
        out = torch.empty((kv.batch, kv.query_heads, kv.head_dim), dtype=torch.float32, device=query.device)
    nbytes = lib().sa_hip_attention_workspace_bytes(kv.batch, kv.query_heads, kv.kv_heads, kv.head_dim, splits)
    if workspace is None and nbytes:
        workspace = torch.zeros(nbytes // 4, dtype=torch.float32, device=query.device)
    s = kv.struct()
    check(lib().sa_hip_sparse_decode_attention(
        C.byref(s), _ptr(query), _ptr(selected), _ptr(counts), select_groups, sel_stride, C.c_float(scale),
        _ptr(out), _ptr(workspace) if nbytes else None, nbytes, splits, _ptr(status), _stream(stream)),
        "sparse_decode_attention")
    return out


def sparse_decode_attention_chunked(kv: PagedKV, query, selected, counts, scale, chunk_pages, max_chunks, out=None,
                                    workspace=None, status=None, stream=None):
    """Attention with every page list cut into chunks of chunk_pages pages
    (one workgroup each, merged): for mixed lengths and budgets.  The default
    workspace has room for the longest-first schedule; one of
    sa_hip_attention_workspace_bytes(..., max_chunks) bytes keeps the grid
    order (same results)."""
    import torch
    select_groups, sel_stride = selected.shape[1], selected.shape[2]
    if out is None:
        out = torch.empty((kv.batch, kv.query_heads, kv.head_dim), dtype=torch.float32, device=query.device)
    if workspace is None:  # room for the partial records and the longest-first schedule
        nbytes = lib().sa_hip_attention_chunked_workspace_bytes(kv.batch, kv.query_heads, kv.kv_heads, kv.head_dim,
                                                                max_chunks)
        workspace = torch.zeros(nbytes // 4, dtype=torch.float32, device=query.device)
    nbytes = workspace.numel() * workspace.element_size()
    s = kv.struct()
    check(lib().sa_hip_sparse_decode_attention_chunked(
        C.byref(s), _ptr(query), _ptr(selected), _ptr(counts), select_groups, sel_stride, C.c_float(scale),
        _ptr(out), _ptr(workspace), nbytes, chunk_pages, max_chunks, _ptr(status), _stream(stream)),
        "sparse_decode_attention_chunked")
    return out


def sparse_decode_attention_partial(kv: PagedKV, query, selected, counts, scale, include_tail, workspace,
                                    split_base, splits, total_splits, status=None, stream=None):
    """Partial records [split_base, split_base + splits) of total_splits."""
    select_groups, sel_stride = selected.shape[1], selected.shape[2]
    s = kv.struct()
    nbytes = workspace.numel() * workspace.element_size()
    check(lib().sa_hip_sparse_decode_attention_partial(
        C.byref(s), _ptr(query), _ptr(selected), _ptr(counts), select_groups, sel_stride, C.c_float(scale),
        1 if include_tail else 0, _ptr(workspace), nbytes, split_base, splits, total_splits, _ptr(status),
        _stream(stream)), "sparse_decode_attention_partial")


def attention_merge(kv: PagedKV, workspace, total_splits, out, stream=None):
    s = kv.struct()
    nbytes = workspace.numel() * workspace.element_size()
    check(lib().sa_hip_attention_merge(C.byref(s), _ptr(workspace), nbytes, total_splits, _ptr(out),
                                       _stream(stream)), "attention_merge")
    return out


def attention_contiguous(kv16, query, tokens, query_heads, kv_heads, scale, out=None, head_dim=HEAD_DIM,
                         stream=None):
    import torch
    if out is None:
        out = torch.empty((query_heads, head_dim), dtype=torch.float32, device=query.device)
    nbytes = lib().sa_hip_contiguous_workspace_bytes(tokens, query_heads, kv_heads, head_dim)
    ws = torch.zeros(max(nbytes // 4, 1), dtype=torch.float32, device=query.device)
    check(lib().sa_hip_attention_contiguous(_ptr(kv16), _ptr(query), tokens, query_heads, kv_heads, head_dim,
                                            C.c_float(scale), _ptr(out), _ptr(ws), nbytes, _stream(stream)),
          "attention_contiguous")
    return out


def append_seal(kv: PagedKV, k, v, local_tokens, status=None, stream=None):
    import torch
    s = kv.struct()
    if k.dtype == torch.uint16:
        check(lib().sa_hip_append_seal_f16(C.byref(s), _ptr(k), _ptr(v), local_tokens, _ptr(status),
                                           _stream(stream)), "append_seal_f16")
    else:
        check(lib().sa_hip_append_seal(C.byref(s), _ptr(k), _ptr(v), local_tokens, _ptr(status),
                                       _stream(stream)), "append_seal")


def seal(kv: PagedKV, local_tokens, status=None, stream=None):
    s = kv.struct()
    check(lib().sa_hip_seal(C.byref(s), local_tokens, _ptr(status), _stream(stream)), "seal")


def local_causal_representatives(prompt_queries, kv16, tokens, query_heads, kv_heads, window, topk, values=True,
                                 offsets=True, reps=None, rep_stride=0, received=None, workspace=None, stream=None,
                                 head_dim=HEAD_DIM, block_tokens=PAGE_TOKENS):
    """InfLLM local-causal block representatives of a prefill (the
    reference's build_local_causal_representatives).  prompt_queries: fp32
    [query_heads, tokens, head_dim]; kv16: uint16 [tokens, 2, kv_heads,
    head_dim].  Returns (values [hq, blocks, head_dim] or None, offsets int32
    [hq, blocks, topk] or None), blocks = tokens // block_tokens; reps
    (optional) is filled in the d-major layout.  workspace: a device tensor
    of at least sa_hip_local_causal_workspace_bytes (allocated here when
    None)."""
    import torch
    dev = prompt_queries.device
    blocks = tokens // block_tokens
    vals = torch.empty((query_heads, blocks, head_dim), dtype=torch.float32, device=dev) if values else None
    offs = torch.empty((query_heads, blocks, topk), dtype=torch.int32, device=dev) if offsets else None
    nbytes = lib().sa_hip_local_causal_workspace_bytes(tokens, query_heads, window)
    if workspace is None:
        ws = torch.empty(max(nbytes // 4, 1), dtype=torch.float32, device=dev)
    else:
        ws = workspace
        nbytes = ws.numel() * ws.element_size()
    check(lib().sa_hip_local_causal_representatives(
        _ptr(prompt_queries), _ptr(kv16), tokens, query_heads, kv_heads, head_dim, block_tokens, window, topk,
        _ptr(vals), _ptr(offs), _ptr(reps), rep_stride, _ptr(received), _ptr(ws), nbytes, _stream(stream)),
        "local_causal_representatives")
    return vals, offs


def gather_pages(pool, page_bytes, num_pages, pages, out, status=None, stream=None):
    check(lib().sa_hip_gather_pages(_ptr(pool), page_bytes, num_pages, _ptr(pages), pages.numel(), _ptr(out),
                                    _ptr(status), _stream(stream)), "gather_pages")
    return out


def read_step_bytes(kv: PagedKV, selected, counts, select_groups, out=None, status=None, stream=None):
    """The decode step's bytes for each (sequence, KV head) read with no
    arithmetic (representatives of the sealed blocks, the selected pages'
    K/V slices, the tail): a bandwidth reference for the attention kernels.
    Returns the XOR of the 32-bit words read, int32 [batch, kv_heads]."""
    import torch
    if out is None:
        out = torch.zeros((kv.batch, kv.kv_heads), dtype=torch.int32, device=kv.pool.device)
    st = kv.struct()
    check(lib().sa_hip_read_step_bytes(C.byref(st), _ptr(selected), _ptr(counts), select_groups,
                                       selected.shape[-1], _ptr(out), _ptr(status), _stream(stream)),
          "read_step_bytes")
    return out


def consume_checksum(x, out, stream=None):
    check(lib().sa_hip_consume_checksum(_ptr(x), x.numel(), _ptr(out), _stream(stream)), "consume_checksum")
    return out


def fill_synthetic_f16(t, seed, first_index=0, stream=None):
    check(lib().sa_hip_fill_synthetic_f16(_ptr(t), t.numel(), seed, first_index, _stream(stream)),
          "fill_synthetic_f16")
    return t


def fill_synthetic_f32(t, seed, first_index=0, stream=None):
    check(lib().sa_hip_fill_synthetic_f32(_ptr(t), t.numel(), seed, first_index, _stream(stream)),
          "fill_synthetic_f32")
    return t


def compare_prediction(predicted, oracle_set):
    """Host set logic of the reference's compare_prediction."""
    import numpy as np
    n = len(predicted)
    p = np.ascontiguousarray(predicted, np.int32)
    o = np.ascontiguousarray(oracle_set, np.int32)
    misses = np.zeros(max(n, 1), np.int32)
    slots = np.zeros(max(n, 1), np.int32)
    hits = C.c_int32(0)
    mc = C.c_int32(0)
    rc = lib().sa_hip_compare_prediction(p.ctypes.data_as(_P), o.ctypes.data_as(_P), n, C.byref(hits),
                                         misses.ctypes.data_as(_P), slots.ctypes.data_as(_P), C.byref(mc))
    check(rc, "compare_prediction")
    return hits.value, misses[: mc.value].tolist(), slots[: mc.value].tolist()


def fill_pages_async(pool, page_bytes, dst_pages, src_base_ptr, src_blocks, copy_stream, done_event=None):
    import numpy as np
    d = np.ascontiguousarray(dst_pages, np.int32)
    s = np.ascontiguousarray(src_blocks, np.int64)
    ev = None if done_event is None else C.c_void_p(done_event.cuda_event)
    check(lib().sa_hip_fill_pages_async(_ptr(pool), page_bytes, d.ctypes.data_as(_P), C.c_void_p(src_base_ptr),
                                        s.ctypes.data_as(_P), len(d), C.c_void_p(copy_stream.cuda_stream), ev),
          "fill_pages_async")


def fill_pages_gather_async(pool, page_bytes, num_pages, dst_pages_dev, src_base_ptr, src_total, src_blocks_dev,
                            count, copy_stream, done_event=None, status=None):
    ev = None if done_event is None else C.c_void_p(done_event.cuda_event)
    check(lib().sa_hip_fill_pages_gather_async(_ptr(pool), page_bytes, num_pages, _ptr(dst_pages_dev),
                                               C.c_void_p(src_base_ptr), src_total, _ptr(src_blocks_dev), count,
                                               _ptr(status), C.c_void_p(copy_stream.cuda_stream), ev),
          "fill_pages_gather_async")


def stream_wait_event(stream, event):
    check(lib().sa_hip_stream_wait_event(C.c_void_p(stream.cuda_stream), C.c_void_p(event.cuda_event)),
          "stream_wait_event")
