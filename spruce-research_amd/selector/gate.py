"""Flat selector gate (inference) on gfx950.

Drop-in for the reference's ``FlatGate`` (selector/gate.py:16-175) on the
scoring path: the same constructor, parameters (``Wq``, ``Wk`` of shape
``[L, d, p]``, kaiming-uniform like nn.Linear) and
``forward(q_feat [L,G,qb,P,d], k_feat [L,G,kb,P,d]) -> [L,G,qb,kb]``
MaxSim scores divided by sqrt(p).  Projection and scoring run as HIP kernels.
Training (autograd through the scores) stays with the reference: this module
scores only, and raises if asked for gradients.
"""
import math

import torch
import torch.nn as nn

from selector.select import gate_scores, project


class FlatGate(nn.Module):
    def __init__(self, num_layers, head_dim, proj_dim=None):
        super().__init__()
        d = head_dim
        p = proj_dim or head_dim
        self.proj_dim = p
        self.Wq = nn.Parameter(torch.empty(num_layers, d, p))
        self.Wk = nn.Parameter(torch.empty(num_layers, d, p))
        for W in (self.Wq, self.Wk):
            nn.init.kaiming_uniform_(W, a=math.sqrt(5))

    def _check_grad(self):
        if torch.is_grad_enabled() and (self.Wq.requires_grad or self.Wk.requires_grad):
            raise RuntimeError("the HIP FlatGate scores only; run it under torch.no_grad()")

    @torch.no_grad()
    def project_queries(self, q_feat):
        """[L,G,qb,P,d] -> [L,G,qb,P,p] (selector/gate.py:120-122)."""
        return torch.stack([project(q_feat[l].float(), self.Wq[l].float()) for l in range(q_feat.shape[0])])

    @torch.no_grad()
    def project_keys(self, k_feat):
        """[L,G,kb,P,d] -> [L,G,kb,P,p] (selector/gate.py:124-127)."""
        return torch.stack([project(k_feat[l].float(), self.Wk[l].float()) for l in range(k_feat.shape[0])])

    def forward(self, q_feat, k_feat, causal=False):
        """Raw MaxSim scores ``[L,G,qb,kb]`` / sqrt(p); ``causal`` sets j > i to -inf."""
        self._check_grad()
        with torch.no_grad():
            qp = self.project_queries(q_feat)
            kp = self.project_keys(k_feat)
            L, G, qb, Pq, p = qp.shape
            kb, Pk = kp.shape[2], kp.shape[3]
            s = gate_scores(qp.reshape(L * G, qb, Pq, p), kp.reshape(L * G, kb, Pk, p),
                            causal=causal, div=math.sqrt(self.proj_dim))
        return s.reshape(L, G, qb, kb)
