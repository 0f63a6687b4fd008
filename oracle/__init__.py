"""CPU oracle for the paged-KV hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import this
package, and only as the checker (or the timed CPU baseline), never as the thing measured or
shipped.  Nothing in ``ecahlang_amd`` imports it: the product path runs the HIP kernels or
raises.

Modules
  manager_ref  -- list-semantics restatement of the reference's AutoKVCacheManager page pool
                  (ecahlang/manager.py:13-253).
  kv_ref       -- numpy restatement of the FlashInfer contract the reference calls:
                  get_seq_lens, get_batch_indices_positions, the append scatter, and
                  gather-then-softmax attention for decode and causal ragged prefill; plus the
                  reference's CPU path (gather pages, then torch SDPA) used as the CPU baseline.
  rope_ref     -- the model's rotary embedding (apply_rotary_pos_emb) with its per-op rounding.
  sampling_ref -- the top-k / top-p sampler's rule.

How each function is pinned (tests/test_oracle_*.py):
  manager_ref      hand-derived traces (tests/golden/manager_traces.json) and invariants.
  seq_lens         closed-form known answers (tests/golden/metadata_kat.json).
  batch_positions  the known answer derived from FlashInfer's documented formula
                   (tests/golden/metadata_kat.json).
  append           brute-force per-element loop on tiny inputs; bitwise pool comparison.
  rope_ref         bitwise against the installed transformers function on CPU; closed forms.
  sampling_ref     closed forms (tests/test_oracle_sampling.py).
  decode / prefill exact special cases (L=1 gives v0, constant V, identical keys give mean V,
                   page-permutation invariance, duplicated KV heads = MHA), a hand-computed
                   2-token example, and agreement with torch SDPA (a library routine).
The reference publishes no golden vectors or tests for this path; FlashInfer's own rounding
and split order are not pinned (they need not be: parity is to a tolerance).
"""
