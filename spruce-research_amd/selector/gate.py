"""Flat selector gate (inference) on gfx950.

Drop-in for the reference's ``FlatGate`` (selector/gate.py:16-175) on the
scoring path: the same constructor, parameters (``Wq``, ``Wk`` of shape
``[L, d, p]``, kaiming-uniform like nn.Linear) and
``forward(q_feat [L,G,qb,P,d], k_feat [L,G,kb,P,d]) -> [L,G,qb,kb]``
MaxSim scores divided by sqrt(p), and the traversal's candidate scoring
(``score_projected_candidates``, ``score_candidates``).  Projection and
scoring run as HIP kernels.
Training (autograd through the scores) stays with the reference: this module
scores only, and raises if asked for gradients.
"""
import math

import torch
import torch.nn as nn

import spruce_hip
from selector.select import gate_scores, project, project_levels


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

    @staticmethod
    def _project(feat, W):
        """``[L, ..., d] -> [L, ..., p]`` float32; 16-bit features are read as they
        are (widened exactly in the kernel), float32 ones directly."""
        def one(x, w):
            if x.dtype in (torch.bfloat16, torch.float16) and x.shape[-1] % 4 == 0 and w.shape[-1] % 4 == 0:
                rows = x.reshape(1, -1, 1, x.shape[-1])
                return project_levels([rows], w).reshape(x.shape[:-1] + (w.shape[-1],))
            return project(x.float(), w.float())
        if feat.shape[0] == 1:
            return one(feat[0], W[0]).unsqueeze(0)
        return torch.stack([one(feat[l], W[l]) for l in range(feat.shape[0])])

    @torch.no_grad()
    def project_key_levels(self, level_features, interleaved=False):
        """Projects the levels of a key tree (each ``[L,G,n_v,P,d]``) into one
        table ``[L,G,sum n_v,P,p]`` with node IDs leaf-first: the values of
        ``project_keys(torch.cat(level_features, dim=2))`` without the copy.
        ``interleaved=True``: the same values as ``[L,G,N,p/4,P,4]`` (the
        traversal's fast key layout)."""
        first = level_features[0]
        L, G, _, P, d = first.shape
        if first.dtype not in (torch.bfloat16, torch.float16, torch.float32) or d % 4 or self.proj_dim % 4:
            out = self.project_keys(torch.cat(level_features, dim=2))
            if interleaved:
                out = out.reshape(out.shape[:4] + (self.proj_dim // 4, 4)).transpose(3, 4).contiguous()
            return out
        outs = []
        for l in range(L):
            outs.append(project_levels([f[l] for f in level_features], self.Wk[l], interleaved=interleaved))
        out = outs[0].unsqueeze(0) if L == 1 else torch.stack(outs)
        return out

    @torch.no_grad()
    def project_queries(self, q_feat):
        """[L,G,qb,P,d] -> [L,G,qb,P,p] (selector/gate.py:120-122)."""
        return self._project(q_feat, self.Wq)

    @torch.no_grad()
    def project_keys(self, k_feat):
        """[L,G,kb,P,d] -> [L,G,kb,P,p] (selector/gate.py:124-127)."""
        return self._project(k_feat, self.Wk)

    @torch.no_grad()
    def score_projected_candidates(self, projected_q, projected_k, candidate_ids, layer_chunk=1):
        """Scores ``[L,G,qb,C]`` of per-row candidate node IDs ``[L,G,qb,C]``
        (clamped to the node range) against projected prototypes
        (selector/gate.py:129-166); one HIP launch, no gathered candidates."""
        if projected_q.dim() != 5 or projected_k.dim() != 5 or candidate_ids.dim() != 4:
            raise ValueError("candidate scoring expects q/k 5-D and IDs 4-D")
        L, G, qb = projected_q.shape[:3]
        if projected_k.shape[:2] != (L, G) or candidate_ids.shape[:3] != (L, G, qb):
            raise ValueError("candidate scoring layer/group/query dimensions mismatch")
        if layer_chunk < 1:
            raise ValueError("layer_chunk must be >= 1")
        if not projected_q.is_cuda:
            raise RuntimeError("the HIP FlatGate requires GPU tensors")
        qp = projected_q.float().contiguous()
        kp = projected_k.float().contiguous()
        ids = candidate_ids.to(torch.int32).contiguous()
        N, Pk, p = kp.shape[2:]
        C = ids.shape[-1]
        out = torch.empty((L, G, qb, C), device=qp.device, dtype=torch.float32)
        if C == 0:
            return out
        with torch.cuda.device(qp.device):
            rc = spruce_hip.lib().spruce_gate_candidate_scores(
                spruce_hip.ptr(qp), spruce_hip.ptr(kp), spruce_hip.ptr(ids), L * G, qb, N, C,
                qp.shape[3], Pk, p, float(math.sqrt(self.proj_dim)), spruce_hip.ptr(out),
                spruce_hip.stream_of(qp))
        spruce_hip.check(rc, "spruce_gate_candidate_scores")
        return out

    @torch.no_grad()
    def score_candidates(self, q_feat, k_feat, candidate_ids):
        """Projects Q/K once, then scores the candidates (selector/gate.py:168-172)."""
        return self.score_projected_candidates(
            self.project_queries(q_feat), self.project_keys(k_feat), candidate_ids)

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
