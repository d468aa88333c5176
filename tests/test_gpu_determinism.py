"""GPU: the attention layer chain is deterministic.  Two copies of the same
seeded state (a paged pool with planted blocks, sealed representatives,
fp32 weights), stepped in lockstep through the q/k/v producer, the one-launch
decode step (append, seal across a block boundary, score, select, attend) and
the o-projection, must agree bit for bit after every step: results depend on
the inputs only, not on which workgroup arrives first.  The reference's CPU
pipeline is deterministic (pipeline_main.cpp:1123 compares a serial and a
pipelined run for equality)."""
import argparse

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def bits(t):
    return t.detach().cpu().numpy().view(np.uint8)


def test_layer_chain_bit_identical_over_seal_boundary(hip):
    import bench
    sa = hip
    batch, hq, hkv, ctx, budget, init, local, planted = 16, 16, 8, 2048 - 5, 24, 2, 4, 4
    steps, hidden, D = 12, 1024, 128
    cfg = (1, batch, hq, hkv, ctx, budget, init, local, planted, None)
    args = argparse.Namespace(seed=4242)
    copies = [bench.Layer(sa, torch, cfg, 0, args, steps + 1) for _ in range(2)]

    def rnd(shape, scale, off):
        t = torch.empty(shape, dtype=torch.float32, device="cuda")
        sa.fill_synthetic_f32(t.view(-1), 77 + off, 0)
        return t * scale

    w = dict(inorm=1 + 0.1 * rnd((hidden,), 1.0, 1), wq=rnd((hq * D, hidden), hidden ** -0.5, 2),
             wk=rnd((hkv * D, hidden), hidden ** -0.5, 3), wv=rnd((hkv * D, hidden), hidden ** -0.5, 4),
             qn=1 + 0.1 * rnd((D,), 1.0, 5), kn=1 + 0.1 * rnd((D,), 1.0, 6),
             wo=rnd((hidden, hq * D), (hq * D) ** -0.5, 7))
    h0 = rnd((batch, hidden), 1.0, 8)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    state = []
    for ly in copies:
        ws, _ = sa.decode_step_workspace(ly.kv, 1)
        state.append(dict(ly=ly, h=h0.clone(), ws=ws, st=torch.zeros(1, dtype=torch.int32, device="cuda"),
                          q=torch.empty((batch, hq, D), dtype=torch.float32, device="cuda"),
                          k=torch.empty((batch, hkv, D), dtype=torch.float32, device="cuda"),
                          v=torch.empty((batch, hkv, D), dtype=torch.float32, device="cuda")))
    sealed0 = int(copies[0].kv.sealed.min().item())
    for s in range(steps):
        for c in state:
            ly = c["ly"]
            sa.qkv_project(c["h"], w["wq"], w["wk"], w["wv"], w["qn"], w["kn"], ly.kv.seq_len, hq, hkv, q=c["q"],
                           k=c["k"], v=c["v"], input_norm=w["inorm"], input_eps=1e-6)
            sa.decode_step(ly.kv, c["k"], c["v"], 0, c["q"], hkv, budget, init, local, scale, c["ws"],
                           selected=ly.selected, counts=ly.counts, out=ly.out, splits=1, status=c["st"])
            c["h"] = sa.linear(ly.out.view(batch, hq * D), w["wo"], c["h"])
        torch.cuda.synchronize()
        a, b = state
        for name in ("q", "k", "v", "h"):
            assert np.array_equal(bits(a[name]), bits(b[name])), (s, name)
        la, lb = a["ly"], b["ly"]
        assert np.array_equal(bits(la.counts), bits(lb.counts)), s
        cnt = la.counts.cpu().numpy()
        sa_, sb_ = la.selected.cpu().numpy(), lb.selected.cpu().numpy()
        for i in range(batch):
            for g in range(hkv):
                assert sa_[i, g, :cnt[i, g]].tolist() == sb_[i, g, :cnt[i, g]].tolist(), (s, i, g)
        assert np.array_equal(bits(la.out), bits(lb.out)), s
        assert int(a["st"].item()) == 0 and int(b["st"].item()) == 0, s
    # the chain crossed a seal: every sequence sealed a new block, and the
    # pools (pages and representatives) are equal byte for byte
    assert int(copies[0].kv.sealed.min().item()) == sealed0 + 1
    for name in ("pool", "reps", "seq_len", "sealed"):
        assert np.array_equal(bits(getattr(copies[0].kv, name)), bits(getattr(copies[1].kv, name))), name
