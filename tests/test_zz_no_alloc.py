"""rmda_moe_layer_static (the allocation-free layer on the library's static
scratch) against rmda_moe_layer with a caller workspace: bitwise equal
outputs on two calls in a row, the second on a smaller input, so the second
call runs on the scratch the first one left behind.  Also its rejections: a
workspace argument, and a shape whose workspace exceeds the scratch."""
import ctypes

import pytest
import torch

from rmda_moe import _lib, api, configs, inputs

pytestmark = pytest.mark.gpu

STATIC_WS_BYTES = 128 << 20  # RMDA_STATIC_WS_BYTES
ERR_ARG, ERR_CAPACITY = -1, -3


def run_pair(ctx, cfg, seed, packed_too=True):
    print("static layer %s seed %d" % (cfg["name"], seed), flush=True)
    inp = inputs.make_inputs(ctx, cfg, seed=seed)
    shape = inp["shape"]
    assert api.workspace_bytes(shape) <= STATIC_WS_BYTES
    packed = ctx.pack_weights(shape, inp["w_router"], inp["w_gate_up"], inp["w_down"], inp["w_sh_gate_up"],
                              inp["w_sh_down"]) if packed_too else None
    ws = inputs.workspace_for(shape)
    ws.fill_(255)
    ref = torch.full((shape["rows"], shape["d"]), float("nan"), dtype=torch.float16, device="cuda")
    got = torch.full_like(ref, float("nan"))
    if packed is not None:
        ctx.layer(shape, inp["x"], inp["w_router"], inp["bias"], None, None, None, None, ref, ws, packed=packed)
        ctx.layer_static(shape, inp["x"], inp["w_router"], inp["bias"], got, packed=packed)
    else:
        ctx.layer(shape, inp["x"], inp["w_router"], inp["bias"], inp["w_gate_up"], inp["w_down"],
                  inp["w_sh_gate_up"], inp["w_sh_down"], ref, ws)
        ctx.layer_static(shape, inp["x"], inp["w_router"], inp["bias"], got, w_gate_up=inp["w_gate_up"],
                         w_down=inp["w_down"], w_sh_gate_up=inp["w_sh_gate_up"], w_sh_down=inp["w_sh_down"])
    ctx.sync()
    assert torch.isfinite(ref.float()).all()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), "static-scratch layer differs"


def test_static_layer_two_calls():
    torch.cuda.set_device(0)
    ctx = api.Context(0)
    try:
        # config 3 (104.7 MB of workspace, the largest benchmark shape that
        # fits), then a smaller ragged call on the scratch it left behind
        run_pair(ctx, configs.CONFIGS[3], seed=0)
        run_pair(ctx, dict(configs.CONFIGS[1], rows=203, name="ragged"), seed=5)
        # HF-layout weights and the shared expert, then config 4 (the hot tile)
        run_pair(ctx, configs.CONFIGS[5] | dict(rows=1024, name="fine_shared_1k"), seed=1, packed_too=False)
        run_pair(ctx, configs.CONFIGS[4], seed=0)
    finally:
        ctx.close()


def test_static_layer_fp32_activations():
    """The static layer with fp32 activations (the slot-scaled mode) against
    rmda_moe_layer with a caller workspace, bitwise, on two calls in a row:
    config 3's shape at 1024 tokens (103.4 MB of workspace in this mode;
    2048 tokens need 188.1 MB, more than the scratch) with activations of
    1e4, then a smaller call of 1e-4 on the scratch the first one left
    behind."""
    torch.cuda.set_device(0)
    ctx = api.Context(0)
    try:
        for cfg, seed, mag in ((dict(configs.CONFIGS[3], rows=1024, name="prefill_1k"), 0, 1e4),
                               (dict(configs.CONFIGS[1], rows=203, name="ragged"), 5, 1e-4)):
            print("static layer x32 %s mag %g" % (cfg["name"], mag), flush=True)
            inp = inputs.make_inputs(ctx, cfg, seed=seed)
            shape = inp["shape"]
            assert api.workspace_bytes_x32(shape) <= STATIC_WS_BYTES
            x32 = inp["x"].float() * mag
            packed = ctx.pack_weights(shape, inp["w_router"], inp["w_gate_up"], inp["w_down"], inp["w_sh_gate_up"],
                                      inp["w_sh_down"])
            ws = torch.full((api.workspace_bytes_x32(shape),), 255, dtype=torch.uint8, device="cuda")
            T, d = shape["rows"], shape["d"]
            hs = [torch.zeros(T, 1, d, dtype=torch.float32, device="cuda") for _ in range(2)]
            inj = torch.zeros(T, 1, dtype=torch.float32, device="cuda")
            ref = torch.full((T, d), float("nan"), dtype=torch.float16, device="cuda")
            got = torch.full_like(ref, float("nan"))
            ctx.layer(shape, None, inp["w_router"], inp["bias"], None, None, None, None, ref, ws, packed=packed,
                      h=hs[0], inj=inj, inj_stride=1, inj_off=0, hc=1, x32=x32)
            ctx.layer_static(shape, None, inp["w_router"], inp["bias"], got, packed=packed, h=hs[1], inj=inj,
                             inj_stride=1, inj_off=0, hc=1, x32=x32)
            ctx.sync()
            assert torch.isfinite(hs[0]).all()
            assert torch.equal(hs[1].view(torch.int32), hs[0].view(torch.int32)), "static-scratch layer differs"
            assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    finally:
        ctx.close()


def test_static_layer_rejections():
    torch.cuda.set_device(0)
    ctx = api.Context(0)
    try:
        cfg = configs.CONFIGS[1]
        inp = inputs.make_inputs(ctx, cfg, seed=0)
        shape = inp["shape"]
        out = torch.empty(shape["rows"], shape["d"], dtype=torch.float16, device="cuda")
        # a workspace argument is an error
        s = api.shape_struct(shape)
        ws = inputs.workspace_for(shape)
        args = _lib.LayerArgs(inp["x"].data_ptr(), inp["w_router"].data_ptr(), None, inp["w_gate_up"].data_ptr(),
                              inp["w_down"].data_ptr(), None, None, out.data_ptr(), ws.data_ptr(),
                              ws.numel(), None, None, None, 0, 0, 0)
        rc = ctx.L.rmda_moe_layer_static(ctx.h, ctypes.byref(s), ctypes.byref(args))
        assert rc == ERR_ARG
        ctx.clear_error()
        # config 5 at full size needs more than the static scratch
        big = configs.shape_of(configs.CONFIGS[5])
        assert api.workspace_bytes(big) > STATIC_WS_BYTES
        s = api.shape_struct(big)
        args = _lib.LayerArgs(inp["x"].data_ptr(), inp["w_router"].data_ptr(), None, inp["w_gate_up"].data_ptr(),
                              inp["w_down"].data_ptr(), inp["w_gate_up"].data_ptr(), inp["w_down"].data_ptr(),
                              out.data_ptr(), None, 0, None, None, None, 0, 0, 0)
        rc = ctx.L.rmda_moe_layer_static(ctx.h, ctypes.byref(s), ctypes.byref(args))
        assert rc == ERR_CAPACITY
        assert "static scratch" in ctx.L.rmda_moe_ctx_message(ctx.h).decode()
        ctx.clear_error()
        # the context still works afterwards
        run_pair(ctx, cfg, seed=2)
    finally:
        ctx.close()


def test_static_layer_allocates_nothing_and_captures_in_a_graph():
    """The header's two promises.  (1) The call allocates nothing: the
    device's free bytes are unchanged across repeated static calls.  (2) It
    enqueues only kernels, so it can be captured in a HIP graph: the graph is
    replayed several times, with eager work and synchronisation between the
    replays, and every replay's output equals rmda_moe_layer's bitwise."""
    torch.cuda.set_device(0)
    ctx = api.Context(0)
    try:
        cfg = configs.CONFIGS[2]
        inp = inputs.make_inputs(ctx, cfg, seed=3)
        shape = inp["shape"]
        packed = ctx.pack_weights(shape, inp["w_router"], inp["w_gate_up"], inp["w_down"], inp["w_sh_gate_up"],
                                  inp["w_sh_down"])
        ws = inputs.workspace_for(shape)
        ref = torch.empty(shape["rows"], shape["d"], dtype=torch.float16, device="cuda")
        ctx.layer(shape, inp["x"], inp["w_router"], inp["bias"], None, None, None, None, ref, ws, packed=packed)
        got = torch.full_like(ref, float("nan"))
        ctx.layer_static(shape, inp["x"], inp["w_router"], inp["bias"], got, packed=packed)
        ctx.sync()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
        free0, _ = torch.cuda.mem_get_info()
        for _ in range(5):
            ctx.layer_static(shape, inp["x"], inp["w_router"], inp["bias"], got, packed=packed)
        ctx.sync()
        free1, _ = torch.cuda.mem_get_info()
        assert free1 == free0, "static layer changed the device's free memory: %d -> %d" % (free0, free1)
        # capture on a side stream; the context issues on it during the capture
        s = torch.cuda.Stream()
        graph = torch.cuda.CUDAGraph()
        out_g = torch.full_like(ref, float("nan"))
        ctx.set_stream(s)
        try:
            with torch.cuda.graph(graph, stream=s):
                ctx.layer_static(shape, inp["x"], inp["w_router"], inp["bias"], out_g, packed=packed)
        finally:
            ctx.set_stream(torch.cuda.current_stream())
        for rep in range(4):
            out_g.fill_(float("nan"))  # eager work between replays
            ctx.layer(shape, inp["x"], inp["w_router"], inp["bias"], None, None, None, None, got, ws, packed=packed)
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out_g.view(torch.int16), ref.view(torch.int16)), "graph replay %d" % rep
        del graph
    finally:
        ctx.close()
