"""CPU oracle for the PLM round's dense-linear hot path. TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg import this package,
and only as the checker (or the timed CPU baseline) — never as a product path. The HIP library in
``plm-anon_amd/`` never calls it.

Every function cites the reference lines it restates. Pinning (each is checked in
``tests/test_oracle.py`` against an independent fp64 brute force, closed forms or special cases):

* ``linear``                — pinned (fp64 brute force within one bf16/fp16 ulp, exact small-integer
                              products, one-hot selection, reduction-order independence).
* ``linear_fp32``           — pinned (fp64 brute force, fp32 tolerance).
* ``nucleus_acceptance``    — pinned (fp64 sort-based brute force, one-hot / uniform / p<=0 /
                              proposal-is-max / tie cases).
* ``floor_acceptance``      — pinned (fp64 brute force, closed-form uniform case).
* ``argmax``                — pinned (ties resolve to the lowest index, brute force).
* ``verify``                — composition of the two above; pinned through them.
* ``epilogue``              — pinned (hand-worked rounds: all accepted, none, first rejection).
* ``gated_lora``            — pinned (fp64 numpy restatement within one output step, no gated row /
                              zero B reduce to ``linear``, exact small-integer shards, one-hot
                              shard routing).
* ``epilogue_state``        — the same bookkeeping with the reference's state writes, from the
                              rule's decisions; ``epilogue`` runs through it, so the hand-worked
                              rounds pin it, plus slot / sequence-capacity cases of its own.

The reference ships no tests or golden vectors for this path (it has none at all), so the fixtures
under ``tests/golden/`` are generated from this oracle on seeded inputs.
"""

from .plm_oracle import (  # noqa: F401
    argmax,
    epilogue,
    epilogue_state,
    floor_acceptance,
    gated_lora,
    gated_lora_fp64,
    linear,
    linear_fp32,
    linear_fp64,
    nucleus_acceptance,
    nucleus_margin,
    silu_mul,
    silu_mul_fp64,
    verify,
)
