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
