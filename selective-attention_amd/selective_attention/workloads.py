"""Seeded synthetic workloads for the benchmark configurations.

One shared generator per configuration so that tests, the benchmark and the
parity checks see bit-identical inputs, index tensors included (varlen
offsets, block selections, page tables).  Everything is drawn from a CPU
torch.Generator seeded with `seed`, in a fixed order, then moved to
`device`.  The only exception is the decode KV page pool, which is large
(gigabytes at full size) and is drawn on the device when `device` is a GPU;
its values never influence any index tensor.

Configurations (BASELINE.json "configs"):
  0  SSD scan fwd, fp32: b2 L512 H8 P64 N64 G1 Lc64
  1  SSD scan fwd+bwd, bf16 activations / fp32 state: b8 L4096 H32 P64 N128 G8 Lc256
  2  varlen block-sparse causal attention, bf16: T=65536, H16, D128, 64-blocks
  3  decode step: paged GQA attention (b64, 32q/8kv, D128, 64-token pages)
     + selective state update (H32 P64 N128 G8)
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

SSD_CONFIGS = {
    0: dict(batch=2, seqlen=512, nheads=8, headdim=64, dstate=64, ngroups=1, chunk=64,
            dtype=torch.float32),
    1: dict(batch=8, seqlen=4096, nheads=32, headdim=64, dstate=128, ngroups=8, chunk=256,
            dtype=torch.bfloat16),
}


def ssd_inputs(batch, seqlen, nheads, headdim, dstate, ngroups, dtype=torch.float32, seed=0,
               device="cpu", with_dy=False, **_unused):
    """x~N(0,1); delta_raw = N(0,1)-4 (dt = softplus(.)); A=-exp(U(0,ln16));
    B,C~N(0,1)/sqrt(64); D~N(0,1) per channel (H*P); dy~N(0,1) (fp32, the
    gradient of the fp32 output y)."""
    g = torch.Generator().manual_seed(seed)
    b, L, H, P, N, G = batch, seqlen, nheads, headdim, dstate, ngroups
    x = torch.randn(b, L, H, P, generator=g)
    delta_raw = torch.randn(b, L, H, generator=g) - 4.0
    A = -torch.exp(torch.rand(H, generator=g) * math.log(16.0))
    Bm = torch.randn(b, L, G, N, generator=g) / 8.0
    Cm = torch.randn(b, L, G, N, generator=g) / 8.0
    D = torch.randn(H * P, generator=g)
    out = dict(u=x.to(dtype), delta_raw=delta_raw.to(dtype), A=A, B=Bm.to(dtype),
               C=Cm.to(dtype), D=D)
    if with_dy:
        out["dy"] = torch.randn(b, L, H, P, generator=g)
    return {k: v.to(device) for k, v in out.items()}


def ssu_inputs(batch=64, nheads=32, headdim=64, dstate=128, ngroups=8, dtype=torch.bfloat16,
               seed=0, device="cpu"):
    """Config 3 state update: state~N(0, 0.1^2) fp32; x/dt/B/C as config 0."""
    g = torch.Generator().manual_seed(seed)
    b, H, P, N, G = batch, nheads, headdim, dstate, ngroups
    x = torch.randn(b, H, P, generator=g)
    delta_raw = torch.randn(b, H, generator=g) - 4.0
    A = -torch.exp(torch.rand(H, generator=g) * math.log(16.0))
    Bm = torch.randn(b, G, N, generator=g) / 8.0
    Cm = torch.randn(b, G, N, generator=g) / 8.0
    D = torch.randn(H * P, generator=g)
    h = torch.randn(b, H, P, N, generator=g) * 0.1
    out = dict(u=x.to(dtype), delta_raw=delta_raw.to(dtype), A=A, B=Bm.to(dtype), C=Cm.to(dtype),
               D=D, h=h)
    return {k: v.to(device) for k, v in out.items()}


# ---------------------------------------------------------------------------
# config 2: varlen packing + block selection
# ---------------------------------------------------------------------------
def varlen_lengths(total_tokens=65536, min_len=256, max_len=8192, generator=None):
    """Lengths ~ U[min_len, max_len] until the sum reaches total_tokens; the last
    one is clipped so the packed length is exactly total_tokens."""
    lens = []
    s = 0
    while s < total_tokens:
        n = int(torch.randint(min_len, max_len + 1, (1,), generator=generator).item())
        n = min(n, total_tokens - s)
        lens.append(n)
        s += n
    return lens


def block_selection(lens, nheads, block_size=64, max_blocks=16, generator=None):
    """Per (head, query block): the diagonal block, the previous block and
    min(max_blocks-2, #earlier) distinct earlier blocks of the same sequence,
    sampled uniformly without replacement.  Sorted ascending, padded with -1.

    Query blocks are numbered globally in packing order (sequence by sequence,
    ceil(len/block_size) blocks each); the stored key-block indices are local
    to the query's sequence (block j covers sequence positions
    [j*block_size, (j+1)*block_size)).

    Returns (block_idx int32 (nheads, n_qblk, max_blocks), qblk_seq int32
    (n_qblk,), qblk_local int32 (n_qblk,)).
    """
    nblk = [math.ceil(n / block_size) for n in lens]
    n_qblk = sum(nblk)
    seq_of = torch.empty(n_qblk, dtype=torch.int32)
    loc_of = torch.empty(n_qblk, dtype=torch.int32)
    i = 0
    for s, nb in enumerate(nblk):
        seq_of[i:i + nb] = s
        loc_of[i:i + nb] = torch.arange(nb, dtype=torch.int32)
        i += nb
    idx = torch.full((nheads, n_qblk, max_blocks), -1, dtype=torch.int32)
    extra = max_blocks - 2
    for h in range(nheads):
        for q in range(n_qblk):
            j = int(loc_of[q])
            sel = [j]
            if j >= 1:
                sel.append(j - 1)
            n_earlier = j - 1
            if n_earlier > 0:
                k = min(extra, n_earlier)
                pick = torch.randperm(n_earlier, generator=generator)[:k]
                sel.extend(int(v) for v in pick)
            sel.sort()
            idx[h, q, :len(sel)] = torch.tensor(sel, dtype=torch.int32)
    return idx, seq_of, loc_of


@dataclass
class SparseAttnWorkload:
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    cu_seqlens: torch.Tensor
    block_idx: torch.Tensor
    lens: list


def sparse_attn_inputs(total_tokens=65536, nheads=16, headdim=128, min_len=256, max_len=8192,
                       block_size=64, max_blocks=16, dtype=torch.bfloat16, seed=0, device="cpu"):
    g = torch.Generator().manual_seed(seed)
    lens = varlen_lengths(total_tokens, min_len, max_len, g)
    cu = torch.zeros(len(lens) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lens, dtype=torch.int64), 0).to(torch.int32)
    idx, _, _ = block_selection(lens, nheads, block_size, max_blocks, g)
    T = int(cu[-1])
    q = torch.randn(T, nheads, headdim, generator=g).to(dtype)
    k = torch.randn(T, nheads, headdim, generator=g).to(dtype)
    v = torch.randn(T, nheads, headdim, generator=g).to(dtype)
    return SparseAttnWorkload(q.to(device), k.to(device), v.to(device), cu.to(device),
                              idx.to(device), lens)


# ---------------------------------------------------------------------------
# config 3: paged GQA decode
# ---------------------------------------------------------------------------
@dataclass
class DecodeWorkload:
    q: torch.Tensor            # (b, Hq, D)
    k_pages: torch.Tensor      # (num_pages, Hkv, page_size, D)
    v_pages: torch.Tensor      # (num_pages, Hkv, D, page_size): V stored transposed per page
    page_table: torch.Tensor   # (b, max_pages) int32, -1 padded
    seq_lens: torch.Tensor     # (b,) int32


def decode_inputs(batch=64, nheads_q=32, nheads_kv=8, headdim=128, min_len=1024,
                  max_len=32768, page_size=64, dtype=torch.bfloat16, seed=0, device="cpu"):
    """seq_lens ~ U[min_len, max_len]; every sequence owns ceil(len/page_size)
    pages of a shared pool; the page numbers are a random permutation of the
    pool.  K pages are (num_pages, Hkv, page_size, D), V pages are stored
    transposed, (num_pages, Hkv, D, page_size).  q is drawn on the CPU; the
    K/V pool on `device` (seeded)."""
    g = torch.Generator().manual_seed(seed)
    seq_lens = torch.randint(min_len, max_len + 1, (batch,), generator=g, dtype=torch.int64)
    npages = [math.ceil(int(n) / page_size) for n in seq_lens]
    total = sum(npages)
    max_pages = math.ceil(max_len / page_size)
    perm = torch.randperm(total, generator=g).to(torch.int32)
    table = torch.full((batch, max_pages), -1, dtype=torch.int32)
    o = 0
    for i, n in enumerate(npages):
        table[i, :n] = perm[o:o + n]
        o += n
    q = torch.randn(batch, nheads_q, headdim, generator=g).to(dtype)
    dev = torch.device(device)
    if dev.type == "cuda":
        gd = torch.Generator(device=dev).manual_seed(seed)
        kp = torch.randn(total, nheads_kv, page_size, headdim, generator=gd, device=dev, dtype=dtype)
        vp = torch.randn(total, nheads_kv, headdim, page_size, generator=gd, device=dev, dtype=dtype)
    else:
        kp = torch.randn(total, nheads_kv, page_size, headdim, generator=g).to(dtype)
        vp = torch.randn(total, nheads_kv, headdim, page_size, generator=g).to(dtype)
    return DecodeWorkload(q.to(dev), kp, vp, table.to(dev), seq_lens.to(torch.int32).to(dev))
