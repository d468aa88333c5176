"""CPU: the long-context miss-correction workload's data design, pinned on
the oracle with no GPU.  tests/cpp/correction_check --cpu-plan builds the
store on the host with the oracle's generator (the bits the device fill
writes), plants 16 blocks per KV head as 4 runs of 4 that move one block per
step, seals with the oracle's tail rule and, at every step, runs the oracle's
shared selection (select_shared_blocks, selection.cpp:96-147) with the
step's Hadamard-row queries: the ids must be exactly init + local + the
runs' current blocks, and compare_prediction (pipeline_main.cpp:686-717)
over the steps must give the designed history coverage 99 / 128."""
import json
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "cpp", "correction_check")


@pytest.fixture(scope="module")
def driver(oracle_lib):
    if not os.path.exists(EXE):
        if not os.path.exists(os.path.join(ROOT, "solidattention-repro_amd", "libsa_hip.so")):
            pytest.skip("libsa_hip.so not built")
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "tests", "cpp"), "correction_check"], check=True)
    return EXE


@pytest.mark.parametrize("batch,context,steps,seed", [(2, 16384, 5, 20261201), (3, 32768, 12, 5)])
def test_planted_selection_and_coverage(driver, batch, context, steps, seed):
    r = subprocess.run([driver, "--cpu-plan", "--batch", str(batch), "--context", str(context), "--steps",
                        str(steps), "--warmup", "2", "--seed", str(seed)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    m = json.loads(r.stdout.strip().splitlines()[-1])
    assert m["selection_mismatches"] == 0
    assert m["history_coverage"] == 99 / 128


def test_steps_beyond_a_page_refused(driver):
    """32 appended tokens would seal the tail page during the replay."""
    r = subprocess.run([driver, "--cpu-plan", "--batch", "1", "--context", "16384", "--steps", "30", "--warmup",
                        "2"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 1 and "bad shape" in r.stderr
