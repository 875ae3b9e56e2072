"""CPU restatement of the causal LM's inference (prefill and decode step).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Follows models/causal_lm.py (CausalLM.forward :104-124, step :126-141),
modules/causal_block.py (:73-139), modules/ssm.py (forward :76-154, step
:156-204) and modules/selective_attention.py (forward :177-290, step
:341-415), composed from this package's restatements: ssd.ssd_scan_forward,
ssu.ssu_forward, ssm_io (conv, context, epilogue) and attn.selective_mha_*.
Arithmetic is fp64 on the CPU.  With bf16=True every tensor the bf16 model
stores between two ops (linear outputs, norms, residual sums, conv and
attention outputs, ...) is rounded to bfloat16 at that point, so that the
remaining difference to the GPU model is the arithmetic inside the ops.

Weights come from a state_dict of selective_attention.models.CausalLM.
A key whose gate is dropped (zeroed, below the threshold, past a length) has
log-gate -inf, the reference's compressed-branch semantics.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from . import attn, ssd, ssm_io, ssu

F64 = torch.float64


class LMRef:
    def __init__(self, state_dict, cfg, bf16=True):
        self.sd = {k: v.detach().to("cpu", F64) for k, v in state_dict.items()}
        self.cfg = cfg
        self.bf16 = bf16
        self.inner = 2 * cfg.model_dim
        self.H = self.inner // cfg.head_dim
        self.Ha = cfg.model_dim // cfg.head_dim
        self.bc = cfg.ssm_num_groups * cfg.ssm_state_dim

    # -- helpers ----------------------------------------------------------
    def rnd(self, x):
        return x.to(torch.bfloat16).to(F64) if self.bf16 else x

    def lin(self, x, name, bias=True):
        w = self.sd[name + ".weight"]
        y = x @ w.T
        if bias and (name + ".bias") in self.sd:
            y = y + self.sd[name + ".bias"]
        return self.rnd(y)

    def norm(self, x, name, eps=1e-6):
        y = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * (1 + self.sd[name + ".weight"])
        return self.rnd(y)

    def rope(self, x, pos):
        """x (..., D) with positions broadcast over its leading dims: the
        rotation of modules/rope.py, angles in fp32 as the module computes them."""
        D = x.shape[-1]
        half = D // 2
        inv = 1.0 / (10000 ** (torch.arange(0, half, dtype=torch.float32) / half))
        ang = pos.to(torch.float32).unsqueeze(-1) * inv
        ang = torch.cat([ang, ang], -1).to(F64)
        rot = torch.cat([-x[..., half:], x[..., :half]], -1)
        return self.rnd(x * torch.cos(ang) + rot * torch.sin(ang))

    def log_gate(self, sg, kept, p):
        std = self.sd[p + "mha.score_std_ema"]
        std = std[None, :, None] if sg.dim() == 3 else std[None, :]
        lg = torch.log(sg) * std * self.cfg.attn_log_gate_penalty
        return torch.where(kept, lg, torch.full_like(lg, float("-inf")))

    def ffn(self, x, p):
        a = self.lin(x, p + "ffn.w1")
        c = self.lin(x, p + "ffn.w2")
        return self.lin(self.rnd(a * self.rnd(F.silu(c))), p + "ffn.out")

    def _conv_w(self, p):
        w = self.sd[p + "ssm.conv.weight"]
        return w.reshape(w.shape[0], w.shape[-1]), self.sd[p + "ssm.conv.bias"]

    # -- prefill ------------------------------------------------------------
    def forward(self, input_ids, lengths=None, thresholds=None):
        """logits (b, L, vocab) and the per-block decode state."""
        cfg = self.cfg
        b, L = input_ids.shape
        P, N, G = cfg.head_dim, cfg.ssm_state_dim, cfg.ssm_num_groups
        H, Ha, D = self.H, self.Ha, cfg.head_dim
        lens = torch.full((b,), L, dtype=torch.int64) if lengths is None else lengths.to(torch.int64)
        h = self.rnd(self.sd["embedding.weight"][input_ids])
        states = []
        for i in range(cfg.num_layers):
            p = f"layers.{i}."
            st = {}
            # SSM (modules/ssm.py:98-152)
            n1 = self.norm(h, p + "norm1")
            proj = self.lin(n1, p + "ssm.in_proj")
            hbc, gate, dr = torch.split(proj, [self.inner + 2 * self.bc, self.inner, H], -1)
            w, cb = self._conv_w(p)
            xbc = self.rnd(ssm_io.conv_forward(hbc, w, cb))
            x, B, C = ssm_io.split(xbc, self.inner, self.bc)
            A = -torch.exp(self.sd[p + "ssm.A_log"])
            y, h_last = ssd.ssd_scan_forward(x.reshape(b, L, H, P), A, B.reshape(b, L, G, N),
                                             C.reshape(b, L, G, N), dr, self.sd[p + "ssm.delta_bias"],
                                             None, lens, cfg.ssm_chunk_size, True,
                                             (0.0, float("inf")), F64)
            out = self.rnd(ssm_io.gate_forward(y.reshape(b, L, -1), x, self.sd[p + "ssm.D"], gate))
            h = self.rnd(h + self.lin(out, p + "ssm.out_proj"))
            st["conv_ctx"] = ssm_io.build_conv_ctx(hbc, lengths, w.shape[1], dtype=F64)
            st["h"] = h_last
            # SelectiveMHA (modules/selective_attention.py:197-290)
            n2 = self.norm(h, p + "norm2")
            g = self.rnd(torch.sigmoid(self.lin(n2, p + "mha.gate_proj")))
            sg, og = g[..., :Ha].transpose(1, 2), g[..., Ha:]
            kept = sg > 0
            thr = None if thresholds is None else thresholds[i]
            if thr is not None:
                kept &= sg >= torch.as_tensor(thr, dtype=F64).reshape(-1)[None, :, None]
            kept &= (torch.arange(L)[None, :] < lens[:, None])[:, None, :]
            v = self.lin(n2, p + "mha.v_proj")
            vh = v.reshape(b, L, Ha, D).transpose(1, 2)
            lg = self.log_gate(sg, kept, p)
            if not bool(kept.any()):
                a = v
            else:
                pos = torch.arange(L)
                q = self.rope(self.lin(n2, p + "mha.q_proj").reshape(b, L, Ha, D), pos[:, None])
                k = self.rope(self.lin(n2, p + "mha.k_proj").reshape(b, L, Ha, D), pos[:, None])
                q, k = q.transpose(1, 2), k.transpose(1, 2)
                a = self.rnd(attn.selective_mha_prefill_ref(q, k, vh, lg, lens))
                a = a.transpose(1, 2).reshape(b, L, -1)
                st["kv"] = [(k[r, :, :int(lens[r])], vh[r, :, :int(lens[r])], lg[r, :, :int(lens[r])])
                            for r in range(b)]
            st.setdefault("kv", [(torch.zeros(Ha, 0, D, dtype=F64), torch.zeros(Ha, 0, D, dtype=F64),
                                  torch.zeros(Ha, 0, dtype=F64)) for _ in range(b)])
            h = self.rnd(h + self.lin(self.rnd(a * og), p + "mha.out_proj"))
            h = self.rnd(h + self.ffn(self.norm(h, p + "norm3"), p))
            states.append(st)
        logits = self.lin(self.norm(h, "norm"), "embedding", bias=False)
        return logits, states

    # -- decode step -------------------------------------------------------
    def step(self, tokens, states, positions, thresholds=None):
        """One token per row at `positions` (b,); `states` is updated in place.
        Returns logits (b, vocab)."""
        cfg = self.cfg
        b = tokens.shape[0]
        P, N, G = cfg.head_dim, cfg.ssm_state_dim, cfg.ssm_num_groups
        H, Ha, D = self.H, self.Ha, cfg.head_dim
        h = self.rnd(self.sd["embedding.weight"][tokens])
        for i in range(cfg.num_layers):
            p = f"layers.{i}."
            st = states[i]
            # SSM.step (modules/ssm.py:160-204)
            proj = self.lin(self.norm(h, p + "norm1"), p + "ssm.in_proj")
            hbc, gate, dr = torch.split(proj, [self.inner + 2 * self.bc, self.inner, H], -1)
            w, cb = self._conv_w(p)
            xbc, st["conv_ctx"] = ssm_io.conv_step(hbc, st["conv_ctx"], w, cb)
            x, B, C = ssm_io.split(self.rnd(xbc), self.inner, self.bc)
            A = -torch.exp(self.sd[p + "ssm.A_log"])
            y, st["h"] = ssu.ssu_forward(x.reshape(b, H, P), A, B.reshape(b, G, N),
                                         C.reshape(b, G, N), dr, self.sd[p + "ssm.delta_bias"],
                                         st["h"])
            out = self.rnd(ssm_io.gate_forward(self.rnd(y).reshape(b, -1), x, self.sd[p + "ssm.D"],
                                               gate))
            h = self.rnd(h + self.lin(out, p + "ssm.out_proj"))
            # SelectiveMHA.step (modules/selective_attention.py:373-405)
            n2 = self.norm(h, p + "norm2")
            g = self.rnd(torch.sigmoid(self.lin(n2, p + "mha.gate_proj")))
            sg, og = g[..., :Ha], g[..., Ha:]
            kept = sg > 0
            thr = None if thresholds is None else thresholds[i]
            if thr is not None:
                kept &= sg >= torch.as_tensor(thr, dtype=F64).reshape(-1)[None, :]
            lg = self.log_gate(sg, kept, p)
            q = self.rope(self.lin(n2, p + "mha.q_proj").reshape(b, Ha, D), positions[:, None])
            k = self.rope(self.lin(n2, p + "mha.k_proj").reshape(b, Ha, D), positions[:, None])
            v = self.lin(n2, p + "mha.v_proj").reshape(b, Ha, D)
            outs = []
            for r in range(b):
                K, V, Gt = st["kv"][r]
                K = torch.cat([K, k[r, :, None]], 1)
                V = torch.cat([V, v[r, :, None]], 1)
                Gt = torch.cat([Gt, lg[r, :, None]], 1)
                st["kv"][r] = (K, V, Gt)
                outs.append(attn.selective_mha_decode_ref(q[r:r + 1], K[None], V[None], Gt[None]))
            a = self.rnd(torch.cat(outs, 0)).reshape(b, -1)
            h = self.rnd(h + self.lin(self.rnd(a * og), p + "mha.out_proj"))
            h = self.rnd(h + self.ffn(self.norm(h, p + "norm3"), p))
        return self.lin(self.norm(h, "norm"), "embedding", bias=False)
