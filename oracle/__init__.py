"""The oracle: a CPU restatement of the reference's tiered-KV attention path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` may import anything from this
package, and only as the checker (or, for the CPU baseline, as the thing the
GPU path is timed beside).  The product (``halo_amd``) never imports it and
has no CPU fallback.

Modules and what pins them (checks live in ``tests/test_oracle.py``):

  attention  -- per-chunk attention + LSE merge + chunk walk
                (halo/kv_cache_chunked.py:194-276, 765-964) and the Triton
                kernel's online-softmax update (halo/triton_chunked.py:46-207).
                Pinned by a float64 brute-force softmax, chunk-size and
                permutation invariance, the causal-truncation identity and
                the fully-masked-chunk rule.
  scoring    -- page-mean keys and the q.Kbar chunk scorer with top-k
                (baselines/scorer_ablations.py:133-139, 204-268), the
                closed-form HALOScorer (halo/scorer.py:36-88), the refetcher
                prediction/scheduling (halo/refetcher.py:38-89).  Pinned by
                brute-force ranking on tiny inputs, margin-checked fixtures
                and the reference tests' expected counts.
  kivi       -- per-group quantise/dequantise (baselines/kivi_cache.py:44-78)
                with per-operation rounding in the storage dtype.  Pinned by
                the reference test's error bound, exhaustive code round trips
                and hand-computed cases at rounding boundaries.
  inputs     -- seeded synthetic inputs for the five benchmark workloads.
  torch_path -- the reference's CPU torch op sequence, used only to time the
                CPU baseline beside the GPU path.

Functions that only an import of the reference could pin bit-for-bit (the
exact fp32 bits of torch reductions) are restated to tolerance and marked
"parity unpinned" where they are defined.
"""
