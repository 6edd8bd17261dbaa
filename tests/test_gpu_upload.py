"""Per-layer weight upload from safetensors (rmda_moe_upload_layer): the
packed buffer it builds from a file is bitwise the one rmda_moe_pack_weights
builds from the same tensors already on the device, for bf16 and fp16
expert weights, with and without a shared expert, through both staging
banks; the layer run on uploaded weights equals the layer run on the HF
tensors; malformed layers fail with a message."""
import numpy as np
import pytest
import torch

from gpu_util import dev
from rmda_moe import api, configs, inputs, st

pytestmark = pytest.mark.gpu

PREFIX = "model.language_model.layers.%d.mlp."


@pytest.fixture(scope="module")
def ctx():
    torch.cuda.set_device(0)
    c = api.Context(0)
    yield c
    c.close()


def shapes():
    base = configs.shape_of(configs.CONFIGS[1])                  # d 512, 8 experts, I 1024
    shared = dict(base, rows=64, experts=16, topk=4, inter=256, shared=256)
    return [dict(base, rows=64), shared]


def device_tensors(ts, prefix, shape):
    """The same tensors on the device in the layout rmda_moe_pack_weights takes."""
    E, d, I, S = shape["experts"], shape["d"], shape["inter"], shape["shared"]
    bf = lambda a: (a.astype(np.uint32) << 16).view(np.float32)  # bf16 bits -> fp32, exact
    r = bf(ts[prefix + "gate.weight"][1]).reshape(E, d)
    if S:
        r = np.concatenate([r, bf(ts[prefix + "shared_expert_gate.weight"][1]).reshape(1, d)])
    out = {"w_router": dev(np.ascontiguousarray(r, np.float32)),
           "gu": dev(ts[prefix + "experts.gate_up_proj"][1]),
           "dn": dev(ts[prefix + "experts.down_proj"][1]), "sgu": None, "sdn": None}
    if S:
        out["sgu"] = dev(np.concatenate([ts[prefix + "shared_expert.gate_proj.weight"][1],
                                         ts[prefix + "shared_expert.up_proj.weight"][1]]))
        out["sdn"] = dev(ts[prefix + "shared_expert.down_proj.weight"][1])
    return out


@pytest.mark.parametrize("dtype", ["BF16", "F16"])
@pytest.mark.parametrize("which", [0, 1])
def test_upload_equals_device_pack(ctx, tmp_path, dtype, which):
    shape = shapes()[which]
    print("upload %s shape %r" % (dtype, shape), flush=True)
    rng = np.random.default_rng(11 + which)
    layers = {l: st.moe_layer_tensors(PREFIX % l, shape, rng, dtype=dtype) for l in range(3)}
    path = tmp_path / "w.safetensors"
    allt = {}
    for l in layers:
        allt.update(layers[l])
    st.write(str(path), allt)
    with st.SafeTensors(str(path)) as f:
        # three layers through the two staging banks, then wait once
        ups = [ctx.upload_layer(f, PREFIX % l, shape) for l in range(3)]
        ctx.upload_wait()
        for l in range(3):
            t = device_tensors(layers[l], PREFIX % l, shape)
            ref = ctx.pack_weights(shape, t["w_router"], t["gu"], t["dn"], t["sgu"], t["sdn"],
                                   bf16=(dtype == "BF16"))
            ctx.sync()
            assert torch.equal(ups[l].view(torch.int16), ref.view(torch.int16)), "layer %d" % l


def test_layer_on_uploaded_weights(ctx, tmp_path):
    shape = dict(shapes()[1], rows=96)
    cfg = dict(configs.CONFIGS[1], **shape, name="upload")
    inp = inputs.make_inputs(ctx, cfg, seed=3)
    rng = np.random.default_rng(5)
    ts = st.moe_layer_tensors(PREFIX % 0, shape, rng, dtype="F16")
    path = tmp_path / "w.safetensors"
    st.write(str(path), ts)
    t = device_tensors(ts, PREFIX % 0, shape)
    ws = inputs.workspace_for(shape)
    out_hf = torch.empty(shape["rows"], shape["d"], dtype=torch.float16, device="cuda")
    ctx.layer(shape, inp["x"], t["w_router"], None, t["gu"], t["dn"], t["sgu"], t["sdn"], out_hf, ws)
    with st.SafeTensors(str(path)) as f:
        packed = ctx.upload_layer(f, PREFIX % 0, shape)
        ctx.upload_wait()
        out_up = torch.empty_like(out_hf)
        ctx.layer(shape, inp["x"], t["w_router"], None, None, None, None, None, out_up, ws, packed=packed)
        ctx.sync()
    assert torch.isfinite(out_hf.float()).all()
    assert torch.equal(out_up.view(torch.int16), out_hf.view(torch.int16))


def test_upload_into_buffer_in_use(ctx, tmp_path):
    """A rotation that reuses a packed buffer: layers reading buffer P are
    queued on the compute stream, then layer B's weights are uploaded into P
    at once.  The pack kernels that overwrite P wait for the queued layers, so
    every queued call still sees A's weights, and a layer after
    rmda_moe_upload_wait sees B's."""
    shape = dict(shapes()[0], rows=64)
    cfg = dict(configs.CONFIGS[1], **shape, name="reuse")
    inp = inputs.make_inputs(ctx, cfg, seed=4)
    rng = np.random.default_rng(9)
    ta = st.moe_layer_tensors(PREFIX % 0, shape, rng, dtype="F16")
    tb = st.moe_layer_tensors(PREFIX % 1, shape, rng, dtype="F16")
    path = tmp_path / "w.safetensors"
    st.write(str(path), {**ta, **tb})
    ws = inputs.workspace_for(shape)
    outs = [torch.empty(shape["rows"], shape["d"], dtype=torch.float16, device="cuda") for _ in range(3)]
    with st.SafeTensors(str(path)) as f:
        packed = ctx.upload_layer(f, PREFIX % 0, shape)
        ctx.upload_wait()
        ref_a = torch.empty_like(outs[0])
        ctx.layer(shape, inp["x"], None, None, None, None, None, None, ref_a, ws, packed=packed)
        pb = ctx.upload_layer(f, PREFIX % 1, shape)
        ctx.upload_wait()
        ref_b = torch.empty_like(outs[0])
        ctx.layer(shape, inp["x"], None, None, None, None, None, None, ref_b, ws, packed=pb)
        ctx.sync()
        assert not torch.equal(ref_a.view(torch.int16), ref_b.view(torch.int16))
        # many queued calls on P (several ms of work), the last one into outs[0]
        for _ in range(400):
            ctx.layer(shape, inp["x"], None, None, None, None, None, None, outs[1], ws, packed=packed)
        ctx.layer(shape, inp["x"], None, None, None, None, None, None, outs[0], ws, packed=packed)
        ctx.upload_layer(f, PREFIX % 1, shape, packed=packed)
        ctx.upload_wait()
        ctx.layer(shape, inp["x"], None, None, None, None, None, None, outs[2], ws, packed=packed)
        ctx.sync()
    assert torch.equal(outs[0].view(torch.int16), ref_a.view(torch.int16)), "a queued layer saw the new weights"
    assert torch.equal(outs[2].view(torch.int16), ref_b.view(torch.int16)), "the layer after the wait saw old weights"


def test_upload_errors(ctx, tmp_path):
    shape = shapes()[0]
    rng = np.random.default_rng(7)
    ts = st.moe_layer_tensors(PREFIX % 0, shape, rng)
    path = tmp_path / "w.safetensors"
    st.write(str(path), ts)
    with st.SafeTensors(str(path)) as f:
        with pytest.raises(api.MoeError, match="missing"):
            ctx.upload_layer(f, PREFIX % 9, shape)
    ctx.clear_error()
    bad = dict(ts)
    bad[PREFIX % 0 + "experts.down_proj"] = ("BF16", ts[PREFIX % 0 + "experts.down_proj"][1][:, :, :128].copy())
    st.write(str(path), bad)
    with st.SafeTensors(str(path)) as f:
        with pytest.raises(api.MoeError, match="down_proj"):
            ctx.upload_layer(f, PREFIX % 0, shape)
    ctx.clear_error()
