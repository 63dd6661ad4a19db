"""The case __graft_entry__.smoke() runs (a small MoE block until the layer lands)."""

import torch

from refs import MoEOracle, cpu
from oracle import reference as R


def run(dev):
    from sgl_amd_mono.k2 import config as C, synth
    from sgl_amd_mono.k2.ops import MoEOp

    cfg = C.MoEConfig(hidden=1024, n_experts=64, top_k=8, inter=256,
                      router=C.ROUTER_SIGMOID_BIAS, route_scale=2.5,
                      expert_fmt=C.FMT_MXFP4, n_shared=1, shared_inter=256)
    w = synth.make_moe(cfg, 4, 11, dev, norm=True)
    out = MoEOp(cfg, w, 4, norm=True, residual=True)(w.x)
    torch.cuda.synchronize()
    ref, *_ = MoEOracle(w)(w.x, norm=True, residual=True)
    err = R.rel_l2(cpu(out).float(), ref)
    if not err <= 1e-2:
        raise AssertionError(f"smoke: MoE rel-L2 {err:.3e} > 1e-2")
