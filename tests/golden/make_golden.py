"""Write the golden fixtures of the attention path (tests/golden/*.npz).

Expected outputs come from the reference's own CPU kernel
(csrc/src/paged_kernels.cpp), compiled from its source by ``make -C oracle
ref`` into oracle/_ref/.  Inputs are regenerated from a seed with NumPy's
PCG64 (platform independent); each fixture stores the seed, the shapes, the
SHA-256 of the regenerated inputs and the expected output, plus the inputs
themselves when they are small.

Cases
  fp32_mha_decode   the 8-sequence fp32 MHA decode step (one flat call with
                    the T x C mask, the reference backend's call pattern)
  gqa_prefill       GQA 6/2, D=16, bs=4, ragged prompts [7, 2, 5, 1]
                    prefilled in one step (block-diagonal causal mask)
  gqa_decode        GQA 8/2, D=8, bs=4, decode of contexts [5, 9, 1, 16]
  mixed_small       one decode + two prefill chunks (start > 0), GQA 4/2,
                    D=32, bs=8
  masked_rows       a mask with fully masked rows (zeros expected)
  empty_context     C == 0 (zeros expected)

Run:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent
sys.path.insert(0, str(REPO))

from oracle import attention as oa  # noqa: E402
from oracle import packing as op  # noqa: E402


def sha256(*arrays: np.ndarray) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def paged_case(seed, hq, hkv, d, bs, starts, counts, pool=None, scale=None, value_scale=1.0):
    """Seeded step over a paged pool: returns a dict of reference-ABI inputs."""
    rng = np.random.Generator(np.random.PCG64(seed))
    ctx = [s + c for s, c in zip(starts, counts)]
    need = [-(-c // bs) for c in ctx]
    total = sum(need) if pool is None else pool
    perm = rng.permutation(total)
    lists, off = [], 0
    for n in need:
        lists.append([int(b) for b in perm[off : off + n]])
        off += n
    t = sum(counts)
    q = (rng.standard_normal((1, hq, t, d)) * value_scale).astype(np.float32)
    k = (rng.standard_normal((1, total, bs, hkv, d)) * value_scale).astype(np.float32)
    v = (rng.standard_normal((1, total, bs, hkv, d)) * value_scale).astype(np.float32)
    gather = op.build_slot_mapping(lists, ctx, bs, [0] * len(ctx), ctx)
    mask = op.attention_mask(starts, counts)
    return dict(
        seed=seed, hq=hq, hkv=hkv, d=d, bs=bs, starts=np.asarray(starts, np.int64),
        counts=np.asarray(counts, np.int64), total_blocks=total,
        block_table=op.build_block_tables(lists, ctx)[0], query=q, key_cache=k, value_cache=v,
        gather_slots=gather, mask=mask, scale=np.float32(1.0 / np.sqrt(d) if scale is None else scale),
    )


def fp32_mha_decode_case(seed=0):
    """8 seqs, 8/8 heads, D=64, bs=16, ctx ~ U{16..512}, pool 512 blocks."""
    rng = np.random.Generator(np.random.PCG64(seed))
    ctx = [int(c) for c in rng.integers(16, 512, size=8, endpoint=True)]
    starts = [c - 1 for c in ctx]
    return paged_case(seed + 1000, 8, 8, 64, 16, starts, [1] * 8, pool=512, scale=0.125)


def write(name, case, store_inputs: bool):
    out = oa.paged_attention(case["query"], case["key_cache"], case["value_cache"], 0,
                             case["gather_slots"], case["mask"], float(case["scale"]), kind="reference")
    payload = {k: v for k, v in case.items()
               if store_inputs or k not in ("query", "key_cache", "value_cache", "mask", "gather_slots")}
    payload["input_sha256"] = np.asarray(sha256(case["query"], case["key_cache"], case["value_cache"]))
    payload["expected"] = out
    np.savez_compressed(HERE / f"{name}.npz", **payload)
    print(f"{name}: output {out.shape}, inputs {'stored' if store_inputs else 'regenerated from seed'}")


CASES = {
    "fp32_mha_decode": (lambda: fp32_mha_decode_case(0), False),
    "gqa_prefill": (lambda: paged_case(11, 6, 2, 16, 4, [0, 0, 0, 0], [7, 2, 5, 1], pool=16, scale=0.35), True),
    "gqa_decode": (lambda: paged_case(12, 8, 2, 8, 4, [4, 8, 0, 15], [1, 1, 1, 1], scale=0.35), True),
    "mixed_small": (lambda: paged_case(13, 4, 2, 32, 8, [20, 5, 17], [1, 6, 9]), True),
}


def masked_rows_case():
    case = paged_case(14, 2, 2, 8, 4, [0, 0], [3, 2], pool=4, scale=0.5)
    case["mask"][0, 0, 1, :] = False  # row 1: nothing attended
    case["mask"][0, 0, 4, :] = False
    return case


def empty_context_case():
    case = paged_case(15, 2, 1, 8, 4, [0], [1], pool=2)
    case["gather_slots"] = np.zeros(0, dtype=np.int64)
    case["mask"] = np.zeros((1, 1, 1, 0), dtype=bool)
    return case


def main():
    if not oa.reference_available():
        raise SystemExit("oracle/_ref is not built: run `make -C oracle ref` with the reference tree present")
    for name, (fn, store) in CASES.items():
        write(name, fn(), store)
    write("masked_rows", masked_rows_case(), True)
    write("empty_context", empty_context_case(), True)


if __name__ == "__main__":
    main()
