"""CPU oracle for the MI355X sampling stage -- TEST INFRASTRUCTURE ONLY.

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import this
package, and only as the checker (or as the timed CPU baseline).  The product path (the HIP library
under `qwen-warp_amd/`) never imports, links or calls it, and fails loudly when its compiled library
is missing.

`oracle.sampler` restates, in PyTorch CPU / numpy / Python integers, the semantics of the
reference's sampling stage (tuan3w/qwen-warp):

  * request logit processors, in the reference order
      engine/src/proc.h:4-5,39-49 (proc_logit), engine/src/proc.cu:8-43 (k_proc_logits),
      engine/src/proc.cu:72-103 (proc_begin gating), tests/test_logit_procs.py:35-62 (ref_rows);
  * the order of candidates: value descending, index ascending
      engine/src/mtp_sample.cu:31-35 (mkkey), engine/src/misc.cu:54 (better);
  * temperature / min_p / top-k / top-p
      engine/src/mtp_sample.cu:150-181 (k_topk2), tests/test_logit_procs.py:239-255 (ref_dist),
      docs/USAGE.md:92-93 (order);
  * Philox4x32-10 draws, key = seed, counter = (position, stream, row key, 0)
      engine/src/mtp_sample.cu:10-27 (philox, rng, u01), engine/src/mtp_sample.h:45 (streams);
  * speculative verification: accept with probability min(1, p/q), else resample from the
      normalised residual max(0, p - q); bonus token from the last row when every draft is accepted
      engine/src/mtp_sample.cu:227-258 (accept_core).

`oracle.pld` restates the reference's prompt-lookup tail proposer (engine/src/pld.cu, engine/include/pld.h);
`oracle/build_ref.sh` builds the reference's own proposer from its sources into `oracle/_ref/` (checker only).

Where the reference's fp32 arithmetic cannot be reproduced bit for bit by any other implementation
(CUDA's expf, warp-order fp32 sums), this oracle fixes an exact integer formulation instead:
fixed-point weights aligned to absolute powers of two, exact integer sums, exact integer
comparisons.  `oracle.sampler`'s module docstring states the definition.
"""
