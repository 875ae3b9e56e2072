"""Write tests/golden/workload_hashes.json: sha256 of the seeded index tensors
(varlen offsets, block selection, decode lengths and page table) produced by
selective_attention.workloads.  Re-run only when the generator is changed on
purpose; test_workload_generators_are_bit_stable pins them."""
import hashlib
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "selective-attention_amd"))

from selective_attention import workloads  # noqa: E402


def h(t):
    return hashlib.sha256(t.contiguous().numpy().tobytes()).hexdigest()


def main():
    w = workloads.sparse_attn_inputs(total_tokens=65536, nheads=16, headdim=128)
    d = workloads.decode_inputs(batch=64, nheads_q=2, nheads_kv=1, headdim=8, device="cpu")
    out = {"config2_cu_seqlens": h(w.cu_seqlens), "config2_block_idx": h(w.block_idx),
           "config2_lens": w.lens, "config3_seq_lens": h(d.seq_lens),
           "config3_page_table": h(d.page_table)}
    with open(os.path.join(HERE, "workload_hashes.json"), "w") as f:
        json.dump(out, f, indent=1)
    print(out)


if __name__ == "__main__":
    main()
