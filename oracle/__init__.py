"""CPU oracle for the QLLM v11 Phase-Associative-Memory hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package (`qllm2_amd`) imports
this package.  Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline`
leg of `bench.py` may use it, and only as the checker / CPU baseline, never as
the thing that is measured or shipped.

Modules
-------
pam   restatement of the PAM scan (chunked dual form, E3 fused multistate,
      K-loop multistate, recurrent decode) in torch-on-CPU, plus brute-force
      complex128 recurrences that pin it.
ce    restatement of the chunked tied-LM-head cross-entropy and its no-grad
      variants.

Parity pinning (what checks each oracle function, see tests/test_oracle_*.py):
  pam.decay_matrices       closed form prod(gamma+1e-6) brute force, C<=8
  pam.dual_form_block      brute-force complex128 recurrence (T<=C)
  pam.chunked_head         brute-force recurrence with (gamma+1e-6); C=T and
                           C=1 special cases; gamma==1 causal prefix sum
  pam.flash_pam_chunked_head  equals chunked_head (ragged tail incl.)
  pam.multistate_fused     equals multistate_loop (M independent scans summed
                           with rotations); M=1 reduces to chunked_head
  pam.recur_step_additive  numpy textbook outer-product recurrence
  gradients                torch.autograd.gradcheck in float64 and brute-force
                           recurrence autograd
  ce.*                     torch.nn.functional.cross_entropy / logsumexp on
                           the full logits, analytic (softmax-onehot)/denom
"""
