"""Synthetic inputs of a configuration, generated on the device by the
library's fill kernels (the same definition as the CPU oracle's generator)."""
import torch

from . import configs


def make_inputs(ctx, cfg, seed=0, device="cuda"):
    """Device tensors for every input of `cfg` (a dict from configs.CONFIGS)."""
    out = {"shape": configs.shape_of(cfg), "seed": seed}
    for name, shp, dt, stream, std in configs.tensor_specs(cfg):
        t = torch.empty(shp, dtype=torch.float16 if dt == "f16" else torch.float32, device=device)
        ctx.fill_normal(t, stream, seed, std)
        out[name] = t
    out["bias"] = None
    bias = configs.router_bias(cfg, seed)
    if bias is not None:
        out["bias"] = torch.from_numpy(bias).to(device)
    for name in ["w_sh_gate_up", "w_sh_down"]:
        out.setdefault(name, None)
    return out


def to_host(inp):
    """numpy copies (uint16 bit patterns for fp16) for the CPU oracle."""
    host = {"shape": dict(inp["shape"])}
    for k, v in inp.items():
        if k in ("shape", "seed"):
            continue
        if v is None:
            host[k] = None
        elif v.dtype == torch.float16:
            host[k] = v.view(torch.int16).cpu().numpy().view("uint16")
        else:
            host[k] = v.cpu().numpy()
    return host


def workspace_for(shape, device="cuda"):
    from .api import workspace_bytes
    n = workspace_bytes(shape)
    if n == 0:
        raise ValueError("shape rejected by rmda_moe_workspace_bytes: %r" % (shape,))
    return torch.empty(n, dtype=torch.uint8, device=device)
