"""Writes tests/golden/c1_decode.npz (run from the repository root).

The c1 workload (Qwen2-0.5B attention: 14 query heads, 2 kv heads,
head_dim 64, block 16, fp32, batch 4, kv_len {17, 64, 130, 255}, pool 256
blocks, seed 0) with NaN in every slot no sequence reads. The new tokens
are written with the oracle's write, then the oracle decodes. Stored: the
post-write pool, the write inputs, the decode inputs and the decode output.
The decode output is cross-checked against the fp64 brute force before it
is saved.
"""

import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path[:0] = [ROOT, os.path.join(ROOT, "mini-vllm-continuous-batching-lab_amd")]

from benchmarks.paged_decode_workloads import make_case  # noqa: E402
from oracle import brute, paged_ref  # noqa: E402


def main() -> None:
    c = make_case("c1", seed=0, nan_fill=True)
    kc, vc = c.key_cache.clone(), c.value_cache.clone()
    paged_ref.write_to_paged_cache(c.new_key, c.new_value, kc, vc, c.slot_mapping, 16)
    out = paged_ref.decode_from_tables(c.query, kc, vc, c.block_table, c.kv_len, 16)
    bf = brute.decode(c.query.numpy(), kc.numpy(), vc.numpy(), c.block_table.numpy(),
                      c.kv_len.numpy(), 16)
    err = float(np.abs(bf - out.double().numpy()).max())
    assert err < 1e-5, err
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c1_decode.npz")
    np.savez_compressed(
        path,
        key_cache=kc.numpy(), value_cache=vc.numpy(), new_key=c.new_key.numpy(),
        new_value=c.new_value.numpy(), slot_mapping=c.slot_mapping.numpy(),
        query=c.query.numpy(), block_table=c.block_table.numpy(), kv_len=c.kv_len.numpy(),
        block_size=np.int64(16), out=out.numpy(),
    )
    print(path, os.path.getsize(path), "bytes; oracle vs fp64 max err", err)


if __name__ == "__main__":
    main()
