"""The layer driven from C: tests/c/qwen_moe_drive (built by
__graft_entry__.build() with gcc, shaped like the qwen.c forwarders over a
minimal mda_qwen_t) runs the fused layer on packed weights and the
stage-by-stage recording, both into hyper-connection streams.  Its results
must be bitwise those of the same calls made through the Python binding on
the same generated inputs, and the fused layer's must be within the layer
tolerance of the oracle."""
import os
import subprocess

import numpy as np
import pytest
import torch

from gpu_util import MAX_ABS
from oracle import oracle as orc
from rmda_moe import api, inputs

pytestmark = pytest.mark.gpu

DRIVER = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c", "qwen_moe_drive")

CASES = [
    # small: shared expert, 4 streams with the logits at column 3 of 11
    dict(name="small", rows=64, d=512, experts=16, topk=4, inter=256, shared=256, skew=False, hc=4, hc_rank=3,
         pad=11),
    # the teacher's MoE shape and stream layout (src/qwen.c:11-37, src/qwen.h:20-21)
    dict(name="teacher", rows=64, d=2560, experts=512, topk=10, inter=640, shared=640, skew=False, hc=4,
         hc_rank=320, pad=384),
]


@pytest.mark.parametrize("cfg", CASES, ids=[c["name"] for c in CASES])
def test_c_driver_matches_python_binding(tmp_path, cfg):
    if not os.path.exists(DRIVER):
        pytest.fail("tests/c/qwen_moe_drive is not built (run __graft_entry__.build())")
    seed = 6
    out = tmp_path / "h.bin"
    T, d, hc, pad = cfg["rows"], cfg["d"], cfg["hc"], cfg["pad"]
    args = [DRIVER, str(out), str(T), str(d), str(cfg["experts"]), str(cfg["topk"]), str(cfg["inter"]),
            str(cfg["shared"]), str(hc), str(cfg["hc_rank"]), str(pad), str(seed)]
    print("C driver %s" % cfg["name"], flush=True)
    r = subprocess.run(args, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    got = np.fromfile(out, dtype=np.float32).reshape(2, T, hc, d)

    torch.cuda.set_device(0)
    ctx = api.Context(0)
    try:
        inp = inputs.make_inputs(ctx, cfg, seed=seed)
        shape = inp["shape"]
        h0 = torch.empty(T, hc, d, dtype=torch.float32, device="cuda")
        inj = torch.empty(T, pad, dtype=torch.float32, device="cuda")
        ctx.fill_normal(h0, 11, seed, 1.0)
        ctx.fill_normal(inj, 12, seed, 3.0)
        packed = ctx.pack_weights(shape, inp["w_router"], inp["w_gate_up"], inp["w_down"], inp["w_sh_gate_up"],
                                  inp["w_sh_down"])
        h_f = h0.clone()
        ws = inputs.workspace_for(shape)
        ctx.layer(shape, inp["x"], inp["w_router"], None, None, None, None, None, None, ws, packed=packed, h=h_f,
                  inj=inj, inj_stride=pad, inj_off=cfg["hc_rank"], hc=hc)
        q = api.QwenMoe(ctx, shape, inp["w_router"], inp["w_gate_up"], inp["w_down"], inp["w_sh_gate_up"],
                        inp["w_sh_down"], hc=hc, hc_rank=cfg["hc_rank"], inj_stride=pad)
        h_r = h0.clone()
        q.moe_rec(inp["x"].float(), T, inj=inj, h=h_r)
        ctx.sync()
        assert np.array_equal(got[0].view(np.uint32), h_f.cpu().numpy().view(np.uint32)), "fused layer from C"
        assert np.array_equal(got[1].view(np.uint32), h_r.cpu().numpy().view(np.uint32)), "recording from C"
        # and the fused layer's streams against the oracle
        ref = orc.layer(inputs.to_host(inp), tile=16, threads=16)
        gate = 2.0 / (1.0 + np.exp(-inj.cpu().numpy().astype(np.float64)[:, cfg["hc_rank"]:cfg["hc_rank"] + hc] / hc))
        want = h0.cpu().numpy().astype(np.float64) + ref["out"].astype(np.float64)[:, None, :] * gate[:, :, None]
        err = np.abs(got[0].astype(np.float64) - want).max()
        print("  C driver hc max-abs %.3g" % err, flush=True)
        assert err <= 2 * MAX_ABS, err
    finally:
        ctx.close()
