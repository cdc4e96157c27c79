"""Writes tests/golden/dsv4_small.pt: small input/output vectors for both ops.

Inputs are the seeded c0 workload (T=16, H=8) and a T=7, H=16, G=2 sibling
case; outputs come from oracle.torch_ref, the restatement of the reference's
own torch oracle, whose FP8 codes are torch's float8_e4m3fn cast.  The file is
data only (tensors, loadable with torch.load(weights_only=True)).  Regenerate
with:  python tests/golden/make_golden.py
"""
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "flaggems-vllm_amd"), ROOT]

import torch  # noqa: E402

from flaggems_vllm import testing as W  # noqa: E402
from oracle import torch_ref  # noqa: E402

OUT = os.path.join(HERE, "dsv4_small.pt")


def main():
    w = W.make_workload(0)
    used = torch.unique(w.position_ids)
    r = w.clone()
    torch_ref.qnorm_rope_kv_insert(*r.args())
    keep = w.slot_mapping >= 0
    s = W.make_inv_rope_workload(7, 16, 2, seed=21, max_pos=4096)
    f8, f32s = torch_ref.inv_rope_fp8_quant(s.o, s.positions, s.cos_sin_cache, 2, 8)
    p8, packed = torch_ref.inv_rope_fp8_quant(s.o, s.positions, s.cos_sin_cache, 2, 8,
                                              tma_aligned_scales=True)
    data = {
        # main op (c0): cos/sin rows only where positions point
        "main.q": w.q, "main.kv": w.kv, "main.slot_mapping": w.slot_mapping,
        "main.position_ids": w.position_ids, "main.cos_sin_rows": w.cos_sin_cache[used],
        "main.cos_sin_row_ids": used, "main.max_pos": torch.tensor(w.meta["max_pos"]),
        "main.num_blocks": torch.tensor(w.k_cache.shape[0]),
        "main.out.q": r.q,
        "main.out.slot_bytes": r.k_cache.view(-1)[_slot_bytes(w.slot_mapping[keep])],
        "main.out.cache_nonzero": torch.count_nonzero(r.k_cache),
        # sibling
        "inv.o": s.o, "inv.positions": s.positions,
        "inv.cos_sin_rows": s.cos_sin_cache[torch.unique(s.positions)],
        "inv.cos_sin_row_ids": torch.unique(s.positions),
        "inv.out.fp8": f8.contiguous(), "inv.out.scale_f32": f32s.contiguous(),
        "inv.out.fp8_tma": p8.contiguous(), "inv.out.scale_packed": packed.contiguous(),
    }
    torch.save(data, OUT)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


def _slot_bytes(slots, bs=64, stride=64 * 584):
    blk, p = slots // bs, slots % bs
    base = blk * stride
    data = base[:, None] + p[:, None] * 576 + torch.arange(576)
    scale = base[:, None] + bs * 576 + p[:, None] * 8 + torch.arange(8)
    return torch.cat((data, scale), 1)


if __name__ == "__main__":
    main()
