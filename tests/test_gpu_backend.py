"""GPU: the C++ boundary, make_hip_backend() and solidattention/hip_kv.hpp,
exercised by the self-checking driver tests/cpp/backend_check (built by
__graft_entry__.build()).  It reproduces the reference's C0/C1/C2 and
lifecycle drivers with their own acceptance bars (C1 max error 2e-5, cosine
0.999999; C2.1 ids [0,8,13,15], packed bytes exact, selected-vs-dense cosine
0.987693; P1.3b.0 448 seals, tail 32, generation 16)."""
import json
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "cpp", "backend_check")


def test_cpp_backend_check(hip):
    assert os.path.exists(EXE), "tests/cpp/backend_check missing: run __graft_entry__.build()"
    print("case: tests/cpp/backend_check", flush=True)
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=110)
    print(r.stdout[-4000:])
    print(r.stderr[-2000:])
    assert r.returncode == 0, f"backend_check exit {r.returncode}"
    m = json.loads(r.stdout)
    assert m["backend"] == "hip-gfx950"
    assert m["c2_selected_block_ids"] == [0, 8, 13, 15]
    assert m["c2_packed_kv_exact"] is True
    assert m["lifecycle_sealed_blocks"] == 448
    assert m["c1_attention_max_abs_error"] <= 2e-5
    for d in (64, 256):  # any head_dim through make_hip_backend()
        assert m[f"c1_head_dim_{d}_attention_max_abs_error"] <= 2e-5
        assert m[f"c1_head_dim_{d}_consumed_abs_error"] <= 1e-4
        # and through the paged C++ API (SparseDecoder: one launch, the token-row kernel)
        assert m[f"decode_step_fused_head_dim_{d}"] is True
        assert m[f"decode_step_selected_ids_exact_head_dim_{d}"] is True
        assert m[f"decode_step_state_bytes_exact_head_dim_{d}"] is True
        assert m[f"decode_step_max_rel_error_head_dim_{d}"] <= 2e-3
        assert m[f"select_attend_max_rel_error_head_dim_{d}"] <= 2e-3
    assert m["decode_step_fused"] is True
    # the shared selection (one block set per sequence) as one launch through the C++ API
    assert m["decode_step_fused_shared"] is True
    assert m["decode_step_selected_ids_exact_shared"] is True
    assert m["decode_step_state_bytes_exact_shared"] is True
    assert m["decode_step_max_rel_error_shared"] <= 2e-3
    # the producer-fed step through the C++ API, equal to the two calls bit for bit
    assert m["decode_step_qkv_equals_two_calls"] is True


EXE_STORE = os.path.join(ROOT, "tests", "cpp", "store_check")


def test_cpp_store_check(hip):
    """The store tier (solidattention/hip_store.hpp): seal writeback to the
    main store (P1.3b.0: 448 sealed and verified, tail 32, generation 16,
    121,110,528 bytes, commit marker) and ticketed store -> pool prefetch
    with miss correction (P1.0: 346 misses, hit rate 0.80692, 448 verified
    tickets, a stale ticket rejected, resident pages equal to the store)."""
    assert os.path.exists(EXE_STORE), "tests/cpp/store_check missing: run __graft_entry__.build()"
    print("case: tests/cpp/store_check", flush=True)
    r = subprocess.run([EXE_STORE], capture_output=True, text=True, timeout=110)
    print(r.stdout[-4000:])
    print(r.stderr[-2000:])
    assert r.returncode == 0, f"store_check exit {r.returncode}"
    m = json.loads(r.stdout)
    assert m["lifecycle_store_verified_reads"] == 448
    assert m["lifecycle_store_bytes"] == 121110528
    assert m["store_prefetch_miss_blocks"] == 346
    assert m["store_prefetch_verified_tickets"] == 448
    assert m["store_prefetch_stale_ticket_rejected"] is True
