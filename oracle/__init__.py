"""CPU oracle for Butterfly compressed attention -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the algorithm of the reference
(Hmbown/Butterfly) for the compressed-attention hot path:

* ``oracle.topology``  -- staged Butterfly block topology and the
  ``causal_shift`` partner rule (``bna/topology/butterfly.py``), plus the Torch
  layout builder (``bna/torch/attention_wayfinder_permute.py:568-682``).
* ``oracle.attention`` -- routing tables, block-mean summaries, one-shot and
  active-row compressed attention (Torch path,
  ``attention_wayfinder_permute.py:912-1197``), and the two-stream from-cache
  semantics with the online-softmax merge (``bna/mlx/attention.py:304-548``,
  ``1601-1876``) restated in torch.
* ``oracle.cache``     -- the two-pool ``CompressedKVCache`` state machine
  (``bna/mlx/compressed_cache.py``) restated in torch.
* ``oracle.brute``     -- the reference tests' numpy brute force
  (``tests/pytorch/test_compressed_butterfly_attention.py:20-85``).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
may import this package, and only as the checker or the timed CPU baseline.
The product (``butterfly_amd``) never imports it and has no CPU fallback.

Pinning (how each function is checked independently of its own formula):

* topology: known-answer tests from the reference's tests
  (``butterfly_stage_meta(32, 0, causal_shift) == (0, 5)``; causal_shift partner
  ``== b - 2**bit`` or None), the ceil(log2 N)-layer prefix-reachability theorem,
  causality/degree/self-in-row invariants, and brute-force enumeration of the
  role map on small N.
* routing tables: brute-force per-query enumeration on small N.
* summaries: closed form (numpy float64 mean) on ragged lengths.
* attention (fp32): the reference tests' numpy brute force, a dense
  softmax over the explicitly enumerated key set, and golden vectors written by
  the reference's own Torch path (``tests/golden``).
* merge: associativity and equality with one softmax over the union.
* cache: the reference tests' invariants (``tail_start % BS == 0``,
  ``W <= tail_size < W + step + BS``, summaries equal block means) and
  from-cache == active-row equality.
"""
