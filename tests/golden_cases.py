"""Regenerates the inputs of a golden fixture from its stored config and seed."""

import hashlib

import torch


def sha(t):
    return hashlib.sha256(t.detach().cpu().contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


def digests(ns):
    return {k: sha(v) for k, v in sorted(vars(ns).items()) if torch.is_tensor(v)}


def regenerate(meta, device):
    from sgl_amd_mono.k2 import config as C
    from sgl_amd_mono.k2 import synth

    kind = meta["kind"]
    if kind == "moe":
        cfg = C.MoEConfig(**meta["cfg"])
        return synth.make_moe(cfg, meta["rows"], meta["seed"], device, norm=meta["norm"])
    if kind == "indexer":
        cfg = C.IndexerConfig(**meta["cfg"])
        return synth.make_indexer(cfg, len(meta["ctx_len"]), meta["seed"], device, ctx_len=meta["ctx_len"])
    if kind == "mla":
        cfg = C.MlaConfig(**meta["cfg"])
        ns = synth.make_mla(cfg, meta["rows"], meta["seed"], device, residual=True)
        ns.sel[0, -meta["unused_tail"]:] = -1
        return ns
    raise ValueError(kind)


def to_device(ns, device):
    """A copy of a synth namespace with every tensor on `device`."""
    from types import SimpleNamespace

    return SimpleNamespace(**{k: v.to(device) if torch.is_tensor(v) else v for k, v in vars(ns).items()})
