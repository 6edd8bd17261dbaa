"""Helpers shared by the GPU tests: byte-exact host <-> device copies and the
acceptance metrics."""
import numpy as np
import torch


def dev(a):
    """numpy -> device tensor with identical bytes (uint32 -> int32, uint16 -> float16)."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        return torch.from_numpy(a.view(np.int32)).cuda()
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).cuda().view(torch.float16)
    return torch.from_numpy(a).cuda()


def u32(t):
    return t.cpu().numpy().view(np.uint32)


def u16(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def f32(t):
    return t.float().cpu().numpy()


def empty_u32(n, fill=None):
    t = torch.empty(n, dtype=torch.int32, device="cuda")
    if fill is not None:
        t.fill_(np.int32(np.uint32(fill).view(np.int32)))
    return t


def out_metrics(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    max_abs = float(np.abs(got - ref).max()) if got.size else 0.0
    den = float(np.linalg.norm(ref))
    rel_l2 = float(np.linalg.norm(got - ref) / den) if den > 0 else 0.0
    return max_abs, rel_l2


# acceptance tolerance of the layer output (fp16 out, fp32 accumulate)
MAX_ABS = 2e-3
REL_L2 = 1e-3

# oracle layers already computed in this process, keyed by (configuration,
# seed, oracle options): the inputs are a pure function of (configuration,
# seed), so tests in different modules that check the same configuration share
# one multithreaded oracle run
_ORACLE_CACHE = {}


def oracle_layer(inp, cfg, seed, **kw):
    """orc.layer(to_host(inp), **kw), computed once per (cfg, seed, kw).
    For inputs exactly as inputs.make_inputs(ctx, cfg, seed) made them (a test
    that edits them calls orc.layer itself)."""
    from oracle import oracle as orc
    from rmda_moe import inputs

    sel = kw.get("rows_sel")
    key = (tuple(sorted(cfg.items())), seed,
           tuple(sorted((k, v) for k, v in kw.items() if k != "rows_sel")),
           None if sel is None else bytes(np.ascontiguousarray(sel, np.uint32)))
    if key not in _ORACLE_CACHE:
        kw.setdefault("threads", 16)
        _ORACLE_CACHE[key] = orc.layer(inputs.to_host(inp), **kw)
    return _ORACLE_CACHE[key]
