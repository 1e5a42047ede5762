"""Helpers shared by the GPU parity tests (not a test module)."""

from __future__ import annotations

import sys

import torch

from benchmarks.paged_decode_workloads import DecodeCase, make_case
from oracle import paged_ref

DEV = torch.device("cuda")
BITS = {torch.float32: torch.int32, torch.float16: torch.int16, torch.bfloat16: torch.int16}

# Max-abs tolerances of the attention output against the fp32 oracle run
# on the same (rounded) inputs.
TOL = {torch.float32: 1e-5, torch.float16: 1e-2, torch.bfloat16: 2e-2}


def say(*a) -> None:
    """Name the case on stdout before a GPU step (flushed)."""
    print(*a, flush=True, file=sys.stdout)


def bits(t: torch.Tensor) -> torch.Tensor:
    """Bit pattern view (NaN-safe exact comparison)."""
    return t.contiguous().view(BITS[t.dtype])


def to_device(case: DecodeCase) -> DecodeCase:
    return DecodeCase(
        layout=case.layout,
        query=case.query.to(DEV),
        key_cache=case.key_cache.to(DEV),
        value_cache=case.value_cache.to(DEV),
        new_key=case.new_key.to(DEV),
        new_value=case.new_value.to(DEV),
        slot_mapping=case.slot_mapping.to(DEV),
        block_table=case.block_table.to(DEV),
        kv_len=case.kv_len.to(DEV),
    )


def oracle_step(case: DecodeCase):
    """CPU oracle of one decode step: write the new tokens, then decode, in
    fp32 on the case's (already rounded) values. Returns (out, kc, vc)."""
    kc = case.key_cache.detach().cpu().float().clone()
    vc = case.value_cache.detach().cpu().float().clone()
    paged_ref.write_to_paged_cache(case.new_key.cpu().float(), case.new_value.cpu().float(), kc,
                                   vc, case.slot_mapping.cpu(), case.layout.spec.block_size)
    out = paged_ref.decode_from_tables(case.query.cpu().float(), kc, vc, case.block_table.cpu(),
                                       case.kv_len.cpu(), case.layout.spec.block_size)
    return out, kc, vc


def cached_case(name: str, seed: int = 0, dtype=None, nan_fill: bool = True):
    """CPU case + its oracle result, memoised per (name, seed, dtype)."""
    key = (name, seed, dtype, nan_fill)
    if key not in _CACHE:
        c = make_case(name, seed=seed, dtype=dtype, nan_fill=nan_fill)
        _CACHE[key] = (c, oracle_step(c))
    return _CACHE[key]


_CACHE: dict = {}
