"""CPU oracle of the warm partial-recompute prefill path -- TEST INFRASTRUCTURE.

This package restates, on the CPU, what the reference computes on the path the
HIP kernels replace.  It checks the product and is never part of it: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and nothing in ``vlcache_amd`` does.

Modules and how each function is pinned (a check that is not a retyping of the
oracle's own formula):

* ``prefill``   integer host logic: recompute count, image range, slot mapping,
                image-KV slot lists, virtual sub-sequences.  Pinned by hand-derived
                known-answer vectors and invariants (tests/test_oracle_prefill.py).
* ``scatter``   store_kvcache and the image-KV copy as index assignments.  Pinned
                by canary rows, skip of slot -1 and an element loop on tiny inputs.
* ``rope``      inverse frequencies, M-RoPE positions and the re-rotation.  Pinned
                against transformers' Qwen2.5-VL rotary embedding and position
                code (an independent implementation in this image), against a
                float64 complex-number rotation, and by R(a)R(b) = R(a+b).
* ``attention`` varlen paged GQA causal attention in fp32.  Pinned against a
                float64 brute-force loop on tiny shapes, torch SDPA's is_causal
                for sq == sk, and layout invariances (paged == contiguous, block
                permutation, GQA == MHA with repeated heads).

* ``engine``    block pool and step scheduler (text-only).  Pinned by known-answer
                step traces and invariants (tests/test_engine_host.py).
* ``vision``    the vision tower in fp32: window layout, 2-D rotary (with the
                reference's bf16 angles), blocks, merger.  Pinned against
                transformers' Qwen2.5-VL vision tower and layout helpers, a
                hand-derived window layout and a bit-level bf16 rounding
                (tests/test_oracle_vision.py).

The attention arithmetic of the reference lives in the external flash-attn
library (pyproject.toml:18, no version pin, absent here): its exact bf16
rounding is not reproducible, so attention parity is tolerance-based.
"""
