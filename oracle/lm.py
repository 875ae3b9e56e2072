"""CPU restatement of the causal LM's inference (prefill and decode step).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Follows models/causal_lm.py (CausalLM.forward :104-124, step :126-141),
models/seq2seq_lm.py (Seq2SeqLM.forward :130-186, step :188-211),
modules/causal_block.py (:73-139), modules/bi_block.py, modules/cross_block.py,
modules/ssm.py (forward :76-154, step :156-204),
modules/selective_attention.py (forward :177-290, step :341-415) and
modules/cross_selective_attention.py (forward :63-157, step :200-238),
composed from this package's restatements: ssd.ssd_scan_forward,
ssu.ssu_forward, ssm_io (conv, context, epilogue), attn.selective_mha_* and
attn.attn_varlen.
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

    # -- block stages, prefill --------------------------------------------
    def ssm_forward(self, x, p, lengths, h_init=None):
        """SSM.forward (modules/ssm.py:98-152) on the normed input x (b, L, d):
        (out_proj output, decode state {conv_ctx, h})."""
        cfg = self.cfg
        b, L, _ = x.shape
        P, N, G, H = cfg.head_dim, cfg.ssm_state_dim, cfg.ssm_num_groups, self.H
        lens = torch.full((b,), L, dtype=torch.int64) if lengths is None else lengths.to(torch.int64)
        proj = self.lin(x, p + "ssm.in_proj")
        hbc, gate, dr = torch.split(proj, [self.inner + 2 * self.bc, self.inner, H], -1)
        w, cb = self._conv_w(p)
        xbc = self.rnd(ssm_io.conv_forward(hbc, w, cb))
        xx, B, C = ssm_io.split(xbc, self.inner, self.bc)
        A = -torch.exp(self.sd[p + "ssm.A_log"])
        y, h_last = ssd.ssd_scan_forward(xx.reshape(b, L, H, P), A, B.reshape(b, L, G, N),
                                         C.reshape(b, L, G, N), dr, self.sd[p + "ssm.delta_bias"],
                                         h_init, lens, cfg.ssm_chunk_size, True,
                                         (0.0, float("inf")), F64)
        out = self.rnd(ssm_io.gate_forward(y.reshape(b, L, -1), xx, self.sd[p + "ssm.D"], gate))
        st = {"conv_ctx": ssm_io.build_conv_ctx(hbc, lengths, w.shape[1], dtype=F64), "h": h_last}
        return self.lin(out, p + "ssm.out_proj"), st

    def mha_forward(self, x, p, lengths, thr, causal=True):
        """SelectiveMHA.forward in inference (modules/selective_attention.py:
        197-290) on the normed input: (out_proj output, per-row decode cache)."""
        b, L, _ = x.shape
        Ha, D = self.Ha, self.cfg.head_dim
        lens = torch.full((b,), L, dtype=torch.int64) if lengths is None else lengths.to(torch.int64)
        g = self.rnd(torch.sigmoid(self.lin(x, p + "mha.gate_proj")))
        sg, og = g[..., :Ha].transpose(1, 2), g[..., Ha:]
        kept = sg > 0
        if thr is not None:
            kept &= sg >= torch.as_tensor(thr, dtype=F64).reshape(-1)[None, :, None]
        kept &= (torch.arange(L)[None, :] < lens[:, None])[:, None, :]
        v = self.lin(x, p + "mha.v_proj")
        vh = v.reshape(b, L, Ha, D).transpose(1, 2)
        lg = self.log_gate(sg, kept, p)
        kv = [(torch.zeros(Ha, 0, D, dtype=F64), torch.zeros(Ha, 0, D, dtype=F64),
               torch.zeros(Ha, 0, dtype=F64)) for _ in range(b)]
        if not bool(kept.any()):
            a = v
        else:
            pos = torch.arange(L)
            q = self.rope(self.lin(x, p + "mha.q_proj").reshape(b, L, Ha, D), pos[:, None])
            k = self.rope(self.lin(x, p + "mha.k_proj").reshape(b, L, Ha, D), pos[:, None])
            if causal:
                q, k = q.transpose(1, 2), k.transpose(1, 2)
                a = self.rnd(attn.selective_mha_prefill_ref(q, k, vh, lg, lens))
                a = a.transpose(1, 2).reshape(b, L, -1)
                kv = [(k[r, :, :int(lens[r])], vh[r, :, :int(lens[r])], lg[r, :, :int(lens[r])])
                      for r in range(b)]
            else:
                # every kept key of the row, the query's own key unbiased
                a = torch.zeros(b, L, Ha, D, dtype=F64)
                for r in range(b):
                    n = int(lens[r])
                    if n == 0:
                        continue
                    cu = torch.tensor([0, n])
                    a[r, :n] = attn.attn_varlen(q[r, :n], k[r, :n], v.reshape(b, L, Ha, D)[r, :n],
                                                cu, "full", key_bias=lg[r, :, :n])
                a = self.rnd(a).reshape(b, L, -1)
        return self.lin(self.rnd(a * og), p + "mha.out_proj"), kv

    def cross_forward(self, x, ctx, ctx_lengths, p, thr, prefill=True):
        """CrossSelectiveMHA.forward in inference (modules/cross_selective_attention.py:
        97-157): (out_proj output, per-row context cache).  At prefill key 0's gate
        is 1 and the threshold applies; without a cache it does not."""
        b, L, _ = x.shape
        Lc = ctx.shape[1]
        Ha, D = self.Ha, self.cfg.head_dim
        clens = torch.full((b,), Lc, dtype=torch.int64) if ctx_lengths is None \
            else ctx_lengths.to(torch.int64)
        gate = self.rnd(torch.sigmoid(self.lin(ctx, p + "cross_mha.select_gate_proj"))).transpose(1, 2)
        first = torch.arange(Lc) == 0
        if prefill:
            gate = torch.where(first[None, None, :], torch.ones_like(gate), gate)
        kept = (gate > 0) & (torch.arange(Lc)[None, :] < clens[:, None])[:, None, :]
        if prefill and thr is not None:
            kept &= (gate >= torch.as_tensor(thr, dtype=F64).reshape(-1)[None, :, None]) | first
        std = self.sd[p + "cross_mha.score_std_ema"]
        lg = torch.log(gate) * std[None, :, None] * self.cfg.attn_log_gate_penalty
        lg = torch.where(kept, lg, torch.full_like(lg, float("-inf")))
        q = self.lin(x, p + "cross_mha.q_proj").reshape(b, L, Ha, D)
        k = self.lin(ctx, p + "cross_mha.k_proj").reshape(b, Lc, Ha, D)
        v = self.lin(ctx, p + "cross_mha.v_proj").reshape(b, Lc, Ha, D)
        a = torch.zeros(b, L, Ha, D, dtype=F64)
        for r in range(b):
            a[r] = attn.attn_varlen(q[r], k[r], v[r], torch.tensor([0, L]), "cross",
                                    torch.tensor([0, Lc]), key_bias=lg[r])
        out = self.lin(self.rnd(a).reshape(b, L, -1), p + "cross_mha.out_proj")
        return out, [(k[r], v[r], lg[r]) for r in range(b)]

    # -- block stages, decode step ----------------------------------------
    def ssm_step(self, x, st, p):
        """SSM.step (modules/ssm.py:160-204); st updated in place."""
        cfg = self.cfg
        b = x.shape[0]
        P, N, G, H = cfg.head_dim, cfg.ssm_state_dim, cfg.ssm_num_groups, self.H
        proj = self.lin(x, p + "ssm.in_proj")
        hbc, gate, dr = torch.split(proj, [self.inner + 2 * self.bc, self.inner, H], -1)
        w, cb = self._conv_w(p)
        xbc, st["conv_ctx"] = ssm_io.conv_step(hbc, st["conv_ctx"], w, cb)
        xx, B, C = ssm_io.split(self.rnd(xbc), self.inner, self.bc)
        A = -torch.exp(self.sd[p + "ssm.A_log"])
        y, st["h"] = ssu.ssu_forward(xx.reshape(b, H, P), A, B.reshape(b, G, N), C.reshape(b, G, N),
                                     dr, self.sd[p + "ssm.delta_bias"], st["h"])
        out = self.rnd(ssm_io.gate_forward(self.rnd(y).reshape(b, -1), xx, self.sd[p + "ssm.D"], gate))
        return self.lin(out, p + "ssm.out_proj")

    def mha_step(self, x, kv, p, positions, thr):
        """SelectiveMHA.step (modules/selective_attention.py:373-405); kv (per-row
        cached keys, values, log-gates) extended in place."""
        b = x.shape[0]
        Ha, D = self.Ha, self.cfg.head_dim
        g = self.rnd(torch.sigmoid(self.lin(x, p + "mha.gate_proj")))
        sg, og = g[..., :Ha], g[..., Ha:]
        kept = sg > 0
        if thr is not None:
            kept &= sg >= torch.as_tensor(thr, dtype=F64).reshape(-1)[None, :]
        lg = self.log_gate(sg, kept, p)
        q = self.rope(self.lin(x, p + "mha.q_proj").reshape(b, Ha, D), positions[:, None])
        k = self.rope(self.lin(x, p + "mha.k_proj").reshape(b, Ha, D), positions[:, None])
        v = self.lin(x, p + "mha.v_proj").reshape(b, Ha, D)
        outs = []
        for r in range(b):
            K, V, Gt = kv[r]
            K = torch.cat([K, k[r, :, None]], 1)
            V = torch.cat([V, v[r, :, None]], 1)
            Gt = torch.cat([Gt, lg[r, :, None]], 1)
            kv[r] = (K, V, Gt)
            outs.append(attn.selective_mha_decode_ref(q[r:r + 1], K[None], V[None], Gt[None]))
        a = self.rnd(torch.cat(outs, 0)).reshape(b, -1)
        return self.lin(self.rnd(a * og), p + "mha.out_proj")

    def cross_step(self, x, ckv, p):
        """CrossSelectiveMHA.step (:225-238): every context key with its bias."""
        b = x.shape[0]
        Ha, D = self.Ha, self.cfg.head_dim
        q = self.lin(x, p + "cross_mha.q_proj").reshape(b, Ha, D)
        outs = []
        for r in range(b):
            K, V, lg = ckv[r]
            s = torch.einsum("hd,nhd->hn", q[r], K) * D ** -0.5 + lg
            outs.append(torch.einsum("hn,nhd->hd", torch.softmax(s, -1), V))
        a = self.rnd(torch.stack(outs)).reshape(b, -1)
        return self.lin(a, p + "cross_mha.out_proj")

    # -- causal LM -------------------------------------------------------------
    def forward(self, input_ids, lengths=None, thresholds=None):
        """logits (b, L, vocab) and the per-block decode state."""
        h = self.rnd(self.sd["embedding.weight"][input_ids])
        states = []
        for i in range(self.cfg.num_layers):
            p = f"layers.{i}."
            s, st = self.ssm_forward(self.norm(h, p + "norm1"), p, lengths)
            h = self.rnd(h + s)
            a, st["kv"] = self.mha_forward(self.norm(h, p + "norm2"), p, lengths,
                                           None if thresholds is None else thresholds[i])
            h = self.rnd(h + a)
            h = self.rnd(h + self.ffn(self.norm(h, p + "norm3"), p))
            states.append(st)
        return self.lin(self.norm(h, "norm"), "embedding", bias=False), states

    def step(self, tokens, states, positions, thresholds=None):
        """One token per row at `positions` (b,); `states` is updated in place.
        Returns logits (b, vocab)."""
        h = self.rnd(self.sd["embedding.weight"][tokens])
        for i in range(self.cfg.num_layers):
            p = f"layers.{i}."
            st = states[i]
            h = self.rnd(h + self.ssm_step(self.norm(h, p + "norm1"), st, p))
            h = self.rnd(h + self.mha_step(self.norm(h, p + "norm2"), st["kv"], p, positions,
                                           None if thresholds is None else thresholds[i]))
            h = self.rnd(h + self.ffn(self.norm(h, p + "norm3"), p))
        return self.lin(self.norm(h, "norm"), "embedding", bias=False)


class Seq2SeqRef(LMRef):
    """Seq2SeqLM (models/seq2seq_lm.py:130-234): BiBlock encoder, final SSM
    and norms, CrossBlock decoder seeded with the normed encoder state."""

    def group_norm(self, x, name, eps=1e-6):
        """norm3: RMSNorm over state_dim with a (heads, state_dim) weight, on
        the state transposed to (b, head_dim, heads, state_dim); fp32 (no
        bf16 storage point)."""
        xt = x.transpose(1, 2)
        y = xt * torch.rsqrt(xt.pow(2).mean(-1, keepdim=True) + eps) * (1 + self.sd[name + ".weight"])
        return y.transpose(1, 2)

    def encode(self, input_ids, lengths, enc_thr=None):
        h = self.rnd(self.sd["embedding.weight"][input_ids])
        for i in range(self.cfg.num_layers):
            p = f"encoder_layers.{i}."
            s, _ = self.ssm_forward(self.norm(h, p + "norm1"), p, lengths)
            h = self.rnd(h + s)
            a, _ = self.mha_forward(self.norm(h, p + "norm2"), p, lengths,
                                    None if enc_thr is None else enc_thr[i], causal=False)
            h = self.rnd(h + a)
            h = self.rnd(h + self.ffn(self.norm(h, p + "norm3"), p))
        s, st = self.ssm_forward(self.norm(h, "norm1"), "", lengths)
        ctx = self.norm(self.rnd(h + s), "norm2")
        return ctx, self.group_norm(st["h"], "norm3")

    def forward(self, input_ids, lengths, dec_ids, enc_thr=None, thr=None, cross_thr=None,
                prefill=True):
        """Decoder logits (b, dec_len, vocab) and the decoder's decode state."""
        ctx, h0 = self.encode(input_ids, lengths, enc_thr)
        h = self.rnd(self.sd["embedding.weight"][dec_ids])
        states = []
        for i in range(self.cfg.num_layers):
            p = f"decoder_layers.{i}."
            s, st = self.ssm_forward(self.norm(h, p + "norm1"), p, None, h_init=h0)
            h = self.rnd(h + s)
            a, st["kv"] = self.mha_forward(self.norm(h, p + "norm2"), p, None,
                                           None if thr is None else thr[i])
            h = self.rnd(h + a)
            c, st["ckv"] = self.cross_forward(self.norm(h, p + "norm3"), ctx, lengths, p,
                                              None if cross_thr is None else cross_thr[i], prefill)
            h = self.rnd(h + c)
            h = self.rnd(h + self.ffn(self.norm(h, p + "norm4"), p))
            states.append(st)
        return self.lin(self.norm(h, "norm4"), "embedding", bias=False), states

    def step(self, tokens, states, positions, thr=None):
        h = self.rnd(self.sd["embedding.weight"][tokens])
        for i in range(self.cfg.num_layers):
            p = f"decoder_layers.{i}."
            st = states[i]
            h = self.rnd(h + self.ssm_step(self.norm(h, p + "norm1"), st, p))
            h = self.rnd(h + self.mha_step(self.norm(h, p + "norm2"), st["kv"], p, positions,
                                           None if thr is None else thr[i]))
            h = self.rnd(h + self.cross_step(self.norm(h, p + "norm3"), st["ckv"], p))
            h = self.rnd(h + self.ffn(self.norm(h, p + "norm4"), p))
        return self.lin(self.norm(h, "norm4"), "embedding", bias=False)


def rope_rotate(x, pos, base=10000.0):
    """The rotation of modules/rope.py on x (..., seq_len, D) at positions
    pos (seq_len,), angles in fp32 as the module computes them, in the
    dtype of x (differentiable in x)."""
    D = x.shape[-1]
    half = D // 2
    inv = 1.0 / (base ** (torch.arange(0, half, dtype=torch.float32) / half))
    ang = pos.to(torch.float32).unsqueeze(-1) * inv
    ang = torch.cat([ang, ang], -1).to(x.dtype)
    rot = torch.cat([-x[..., half:], x[..., :half]], -1)
    return x * torch.cos(ang) + rot * torch.sin(ang)


def selective_mha_train_forward(params, x, lengths, head_dim, penalty, causal=True):
    """SelectiveMHA's training forward (modules/selective_attention.py:197-277)
    in the dtype of x, differentiable in x and in params: gates =
    sigmoid(gate_proj(x)) split into (heads, dim); q, k, v projections; RoPE
    on q and k; the attention of attn.selective_mha_train_attn (the current
    batch's score std in the log-gate); out_proj(out * out_gate).
    params: gate_proj.weight/.bias, q_proj.weight, k_proj.weight,
    v_proj.weight/.bias, out_proj.weight/.bias.  Returns (hidden (batch,
    seq_len, dim), std (heads,))."""
    b, L, dim = x.shape
    H = dim // head_dim
    g = torch.sigmoid(F.linear(x, params["gate_proj.weight"], params["gate_proj.bias"]))
    sg, og = g[..., :H].transpose(1, 2), g[..., H:]
    heads = lambda t: t.view(b, L, H, head_dim).transpose(1, 2)
    q = heads(F.linear(x, params["q_proj.weight"]))
    k = heads(F.linear(x, params["k_proj.weight"]))
    v = heads(F.linear(x, params["v_proj.weight"], params["v_proj.bias"]))
    pos = torch.arange(L)
    out, std = attn.selective_mha_train_attn(rope_rotate(q, pos), rope_rotate(k, pos), v, sg,
                                             penalty, lengths, causal, dtype=x.dtype)
    out = out.transpose(1, 2).reshape(b, L, dim)
    return F.linear(out * og, params["out_proj.weight"], params["out_proj.bias"]), std


def cross_mha_train_forward(params, x, ctx, ctx_lengths, head_dim, penalty):
    """CrossSelectiveMHA's training forward (modules/cross_selective_attention.py:88-161)
    in the dtype of x, differentiable in x, ctx and params: gate =
    sigmoid(select_gate_proj(ctx)); scores scale * q.k with keys past the
    context length at -inf; the per-head std of the finite scores; log-gate =
    log(gate) * std * penalty added to every key but key 0; softmax; times v;
    out_proj.  params: q_proj.weight, k_proj.weight, v_proj.weight/.bias,
    out_proj.weight/.bias, select_gate_proj.weight/.bias.  Returns (hidden
    (batch, q_len, dim), std (heads,))."""
    b, L, dim = x.shape
    Lc = ctx.shape[1]
    H = dim // head_dim
    heads = lambda t, n: t.view(b, n, H, head_dim).transpose(1, 2)
    sg = torch.sigmoid(F.linear(ctx, params["select_gate_proj.weight"],
                                params["select_gate_proj.bias"])).transpose(1, 2)
    q = heads(F.linear(x, params["q_proj.weight"]), L)
    k = heads(F.linear(ctx, params["k_proj.weight"]), Lc)
    v = heads(F.linear(ctx, params["v_proj.weight"], params["v_proj.bias"]), Lc)
    s = torch.matmul(q, k.transpose(-2, -1)) * head_dim ** -0.5
    if ctx_lengths is not None:
        pad = torch.arange(Lc)[None, :] >= ctx_lengths.to(torch.int64).cpu()[:, None]
        s = s.masked_fill(pad[:, None, None, :], float("-inf"))
    valid = torch.isfinite(s)
    cnt = valid.sum(dim=(0, 2, 3)).to(x.dtype).clamp(min=1)
    sv = torch.where(valid, s, torch.zeros((), dtype=x.dtype))
    mean = sv.sum(dim=(0, 2, 3)) / cnt
    std = ((sv * sv).sum(dim=(0, 2, 3)) / cnt - mean * mean).clamp(min=0).sqrt()
    lg = torch.log(sg) * std[None, :, None] * penalty
    s = torch.cat([s[..., :1], s[..., 1:] + lg[:, :, None, 1:]], dim=-1)
    out = (torch.softmax(s, dim=-1) @ v).transpose(1, 2).reshape(b, L, dim)
    return F.linear(out, params["out_proj.weight"], params["out_proj.bias"]), std
