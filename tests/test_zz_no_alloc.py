"""GPU: the allocation-free decode step (sa_hip_decode_step_noalloc, static
per-GPU scratch) against the decode step with a caller's workspace
(sa_hip_decode_step), which the other decode-step tests hold to the oracle.

Both run on identical copies of the same paged state: page bytes,
representatives, counters and selected ids must be equal bit for bit, the
attention outputs within 2e-3 (the same kernels run, so
they are expected to be equal).  Two calls in a row share the scratch, the
second with a smaller batch and shorter contexts; the unfused launches
(splits 2) keep their split records in the scratch."""
import numpy as np
import pytest
import torch

from gpu_util import assert_close_2e3, device_kv, pool_numpy, status_tensor, to_dev
from paged_case import D, make_case

pytestmark = pytest.mark.gpu

SCALE = float(np.float32(1.0) / np.sqrt(np.float32(128)))
BUDGET, INIT, LOCAL = 16, 2, 3

# two calls in a row: (seed, lengths, table_stride), the second smaller
CALLS = [
    (801, [32 * 40 + 31, 32 * 12 + 5, 32 * 70 + 31, 32 * 3, 32 * 20 + 30], 80),
    (802, [32 * 9 + 31, 32 * 25, 32 * 5 + 2], 40),
]


def outputs(batch, hq):
    sel = torch.full((batch, 8, BUDGET), -1, dtype=torch.int32, device="cuda")
    cnt = torch.full((batch, 8), -1, dtype=torch.int32, device="cuda")
    out = torch.full((batch, hq, D), float("nan"), dtype=torch.float32, device="cuda")
    return sel, cnt, out


def assert_same_state(kv_a, kv_b):
    assert np.array_equal(kv_a.seq_len.cpu().numpy(), kv_b.seq_len.cpu().numpy())
    assert np.array_equal(kv_a.sealed.cpu().numpy(), kv_b.sealed.cpu().numpy())
    assert np.array_equal(kv_a.generation.cpu().numpy(), kv_b.generation.cpu().numpy())
    assert np.array_equal(pool_numpy(kv_a), pool_numpy(kv_b))
    assert np.array_equal(kv_a.reps.cpu().numpy().view(np.uint32), kv_b.reps.cpu().numpy().view(np.uint32))


def assert_same_step(a, b):
    (sel_a, cnt_a, out_a), (sel_b, cnt_b, out_b) = a, b
    ca = cnt_a.cpu().numpy()
    assert np.array_equal(ca, cnt_b.cpu().numpy())
    sa_, sb_ = sel_a.cpu().numpy(), sel_b.cpu().numpy()
    for bb in range(ca.shape[0]):
        for g in range(ca.shape[1]):
            assert sa_[bb, g, : ca[bb, g]].tolist() == sb_[bb, g, : ca[bb, g]].tolist(), (bb, g)
    assert_close_2e3(out_b.cpu().numpy(), out_a.cpu().numpy())


@pytest.mark.parametrize("hq,splits", [(16, (1, 1)), (32, (1, 1)), (16, (2, 2)), (32, (2, 1))])
def test_noalloc_equals_workspace_entry_two_calls(hip, hq, splits):
    for call, ((seed, lengths, stride), sp) in enumerate(zip(CALLS, splits)):
        print(f"case: hq={hq} call={call} batch={len(lengths)} splits={sp}", flush=True)
        case = make_case(seed + hq, len(lengths), hq, 8, lengths, table_stride=stride, planted=3)
        kv_a, kv_b = device_kv(case), device_kv(case)
        assert hip.select_attend_fused(kv_a, 8, sp) == (sp == 1)
        ws, _ = hip.decode_step_workspace(kv_a, sp)
        rng = np.random.default_rng(seed)
        st_a, st_b = status_tensor(), status_tensor()
        for step in range(3):  # the third step of the first call seals a block
            k = to_dev((rng.standard_normal((case.batch, 8, D)) * 2).astype(np.float32))
            v = to_dev((rng.standard_normal((case.batch, 8, D)) * 2).astype(np.float32))
            q = to_dev(rng.standard_normal((case.batch, hq, D)).astype(np.float32))
            a = hip.decode_step(kv_a, k, v, 0, q, 8, BUDGET, INIT, LOCAL, SCALE, ws, splits=sp, status=st_a)
            b = hip.decode_step_noalloc(kv_b, k, v, 0, q, 8, BUDGET, INIT, LOCAL, SCALE, *outputs(case.batch, hq),
                                        splits=sp, status=st_b)
            torch.cuda.synchronize()
            assert int(st_a.item()) == 0 and int(st_b.item()) == 0
            assert_same_step(a, b)
        assert_same_state(kv_a, kv_b)
        assert int(kv_b.sealed.cpu().numpy()[0]) == (32 * 40 + 31 + 3) // 32 or call == 1


@pytest.mark.parametrize("hq,splits", [(16, 1), (32, 1), (16, 2)])
def test_noalloc_shared_selection_two_calls(hip, hq, splits):
    """The shared selection (select_groups 1): in one launch (splits 1) and as
    separate launches whose split selection keeps its scores in the scratch
    (splits 2), two calls in a row, the second smaller, equal to the decode
    step with a workspace."""
    for call, (seed, lengths, stride) in enumerate(CALLS):
        print(f"case: shared hq={hq} call={call} batch={len(lengths)} splits={splits}", flush=True)
        case = make_case(seed + 50 + hq, len(lengths), hq, 8, lengths, table_stride=stride, planted=3)
        kv_a, kv_b = device_kv(case), device_kv(case)
        assert hip.select_attend_fused(kv_a, 1, splits) == (splits == 1)
        ws, _ = hip.decode_step_workspace(kv_a, splits)
        rng = np.random.default_rng(seed + 1)
        st_a, st_b = status_tensor(), status_tensor()
        for step in range(3):
            k = to_dev((rng.standard_normal((case.batch, 8, D)) * 2).astype(np.float32))
            v = to_dev((rng.standard_normal((case.batch, 8, D)) * 2).astype(np.float32))
            q = to_dev(rng.standard_normal((case.batch, hq, D)).astype(np.float32))
            a = hip.decode_step(kv_a, k, v, 0, q, 1, BUDGET, INIT, LOCAL, SCALE, ws, splits=splits, status=st_a)
            sel = torch.full((case.batch, 1, BUDGET), -1, dtype=torch.int32, device="cuda")
            cnt = torch.full((case.batch, 1), -1, dtype=torch.int32, device="cuda")
            out = torch.full((case.batch, hq, D), float("nan"), dtype=torch.float32, device="cuda")
            b = hip.decode_step_noalloc(kv_b, k, v, 0, q, 1, BUDGET, INIT, LOCAL, SCALE, sel, cnt, out, splits=splits,
                                        status=st_b)
            torch.cuda.synchronize()
            assert int(st_a.item()) == 0 and int(st_b.item()) == 0
            assert_same_step(a, b)
        assert_same_state(kv_a, kv_b)


def test_noalloc_refuses_records_beyond_scratch(hip):
    case = make_case(805, 2, 16, 8, [32 * 4 + 1, 32 * 3], table_stride=8)
    kv = device_kv(case)
    big = 1024  # 2 x 8 x 1024 x 2 x 528 B of split records > the scratch
    z = torch.zeros((2, 8, D), dtype=torch.float32, device="cuda")
    with pytest.raises(hip.SaHipError, match="static scratch"):
        hip.decode_step_noalloc(kv, z, z, 0, to_dev(case.query), 8, BUDGET, INIT, LOCAL, SCALE, *outputs(2, 16),
                                splits=big)
    torch.cuda.synchronize()
    assert kv.seq_len.cpu().numpy().tolist() == [32 * 4 + 1, 32 * 3]  # nothing launched


@pytest.mark.parametrize("splits", [1, 2])
def test_noalloc_graph_replays(hip, splits):
    """Captured in a HIP graph and replayed 3 times with eager work between
    replays: every replay equals an eager step of the workspace entry point
    on a copy of the state.  splits 1: the counter clear and the fused step;
    splits 2: the separate append/seal, selection and attention launches,
    whose split records live in the static scratch."""
    print(f"case: graph replays splits={splits}", flush=True)
    case = make_case(806, 4, 16, 8, [32 * 60 + 30, 32 * 33, 32 * 12 + 3, 32 * 70 + 31], table_stride=80, planted=3)
    rng = np.random.default_rng(7)
    k = to_dev((rng.standard_normal((4, 8, D)) * 2).astype(np.float32))
    v = to_dev((rng.standard_normal((4, 8, D)) * 2).astype(np.float32))
    q = to_dev(case.query)
    # the first call on the device (the scratch address lookup) runs eagerly
    warm = device_kv(case)
    hip.decode_step_noalloc(warm, k, v, 0, q, 8, BUDGET, INIT, LOCAL, SCALE, *outputs(4, 16))
    torch.cuda.synchronize()
    kv_a, kv_b = device_kv(case), device_kv(case)
    assert hip.select_attend_fused(kv_a, 8, splits) == (splits == 1)
    ws, _ = hip.decode_step_workspace(kv_a, splits)
    sel, cnt, out = outputs(4, 16)
    st = status_tensor()
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            hip.decode_step_noalloc(kv_b, k, v, 0, q, 8, BUDGET, INIT, LOCAL, SCALE, sel, cnt, out, splits=splits,
                                    status=st)
    torch.cuda.synchronize()
    for r in range(3):
        print(f"replay {r}", flush=True)
        a = hip.decode_step(kv_a, k, v, 0, q, 8, BUDGET, INIT, LOCAL, SCALE, ws, splits=splits)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        _ = (out * 2).sum().item()  # eager work between replays
        assert int(st.item()) == 0
        assert_same_step(a, (sel, cnt, out))
        assert_same_state(kv_a, kv_b)
    assert int(kv_b.seq_len.cpu().numpy()[0]) == 32 * 60 + 30 + 3  # three appends, one seal on the way


FIRST_CALL_UNDER_CAPTURE = r"""
import sys
sys.path.insert(0, {root!r}); sys.path.insert(0, {pkg!r}); sys.path.insert(0, {tests!r})
import numpy as np, torch
import solidattention_amd as sa
from gpu_util import device_kv
from paged_case import make_case
case = make_case(807, 2, 16, 8, [32 * 5 + 3, 32 * 2], table_stride=8)
kv = device_kv(case)
z = torch.zeros((2, 8, 128), dtype=torch.float32, device="cuda")
q = torch.from_numpy(case.query).cuda()
sel = torch.zeros((2, 8, 16), dtype=torch.int32, device="cuda")
cnt = torch.zeros((2, 8), dtype=torch.int32, device="cuda")
out = torch.zeros((2, 16, 128), dtype=torch.float32, device="cuda")
torch.cuda.synchronize()
side = torch.cuda.Stream()
msg = "no error"
try:
    with torch.cuda.stream(side):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            sa.decode_step_noalloc(kv, z, z, 0, q, 8, 16, 2, 3, 0.088, sel, cnt, out)
except Exception as e:  # the capture ends with the refusal
    msg = str(e)
torch.cuda.synchronize()
print("REFUSED" if "outside graph capture" in msg else "NOT REFUSED: " + msg, flush=True)
# and eagerly the same call then works
sa.decode_step_noalloc(kv, z, z, 0, q, 8, 16, 2, 3, 0.088, sel, cnt, out)
torch.cuda.synchronize()
print("EAGER OK", int(kv.seq_len[0].item()), flush=True)
"""


def test_noalloc_first_call_under_capture_refused(hip):
    """In a fresh process (no earlier call on the device), a first call made
    under graph capture is refused with a clear error before anything is
    launched; the same call made eagerly afterwards runs."""
    import os
    import subprocess
    import sys
    here = os.path.dirname(os.path.abspath(__file__))
    root = os.path.dirname(here)
    script = FIRST_CALL_UNDER_CAPTURE.format(root=root, pkg=os.path.join(root, "solidattention-repro_amd"),
                                             tests=here)
    print("case: first noalloc call under capture, fresh process", flush=True)
    r = subprocess.run([sys.executable, "-c", script], capture_output=True, text=True, timeout=110)
    print(r.stdout[-2000:], r.stderr[-2000:])
    assert r.returncode == 0
    assert "REFUSED" in r.stdout and "NOT REFUSED" not in r.stdout
    assert "EAGER OK 164" in r.stdout
