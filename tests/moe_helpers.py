"""Shared GPU-test helpers: a MoE layer uploaded to the device and described to
the CPU oracle (crates/bridge-kernels-reference/src/moe.rs:64-147 semantics)."""
import numpy as np
import torch

from lbhip import synth


def dev(a):
    return torch.from_numpy(np.array(a, copy=True)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


class Layer:
    """One MoE layer uploaded to the GPU and described to the oracle."""

    def __init__(self, be, oracle, n_experts, hidden, ffn_r, ffn_s, types, seed, scale=None):
        gr, dr, gs, ds = types
        self.hidden = hidden
        self.np = []
        dev_exp, orc_exp = [], []
        for e in range(n_experts):
            g = synth.random_matrix(gr, ffn_r, hidden, seed + 7 * e)
            u = synth.random_matrix(gr, ffn_r, hidden, seed + 7 * e + 1)
            d = synth.random_matrix(dr, hidden, ffn_r, seed + 7 * e + 2)
            if scale is not None:
                scale(e, g, u, d)
            self.np.append((g, u, d))
            dev_exp.append((be.upload(gr, ffn_r, hidden, g), be.upload(gr, ffn_r, hidden, u),
                            be.upload(dr, hidden, ffn_r, d)))
            orc_exp.append(oracle.make_expert(oracle.make_matrix(gr, ffn_r, hidden, g),
                                              oracle.make_matrix(gr, ffn_r, hidden, u),
                                              oracle.make_matrix(dr, hidden, ffn_r, d)))
        sg = synth.random_matrix(gs, ffn_s, hidden, seed + 1001)
        su = synth.random_matrix(gs, ffn_s, hidden, seed + 1002)
        sd = synth.random_matrix(ds, hidden, ffn_s, seed + 1003)
        self.shared_np = (sg, su, sd)
        dev_sh = (be.upload(gs, ffn_s, hidden, sg), be.upload(gs, ffn_s, hidden, su), be.upload(ds, hidden, ffn_s, sd))
        self.orc_shared = oracle.make_expert(oracle.make_matrix(gs, ffn_s, hidden, sg),
                                             oracle.make_matrix(gs, ffn_s, hidden, su),
                                             oracle.make_matrix(ds, hidden, ffn_s, sd))
        self.orc_experts = orc_exp
        self.moe = be.moe_create(dev_exp, dev_sh)
        self._keep = (dev_exp, dev_sh)

    def oracle_out(self, oracle, ids, coefs, x, sentinel=None):
        out = np.full(self.hidden, np.nan, np.float32) if sentinel is None else sentinel.copy()
        ex = oracle.make_exec(oracle.MODE_CPU_PARALLEL_Q8K, 8, True)
        err = oracle.moe_routed_by_id_status(ex, ids, coefs, self.orc_experts, self.orc_shared, x, out)
        return out, err
