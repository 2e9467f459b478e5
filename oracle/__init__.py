"""CPU oracle of diff-gpt's attention hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the host, the arithmetic of fxeqxmulfx/diff-gpt's
attention path so that the HIP library can be checked against it:

  oracle.numerics  numpy: bf16/fp16 rounding, the RoPE table, RoPE, the
                   parameter-free RMSNorm in the canonical reduction order of
                   the kernels, fp64 brute-force attention with the reference's
                   three mask branches, and a numpy KV cache with the
                   reference's growth / prefill / pos rules.
  oracle.torch_ref torch on the CPU: the reference model's forward (GPT,
                   Block-AttnRes, gated MHA with F.scaled_dot_product_attention
                   and F.rms_norm) as a function of a state_dict, and the
                   KV-cache decode loop.  Serves the end-to-end parity tests
                   and bench.py's CPU baseline.

Only tests/, __graft_entry__.smoke() and the cpu_baseline leg of bench.py may
import it, and only as the checker / the timed CPU baseline.  The product
package (diff-gpt_amd/diff_gpt) never imports it and has no CPU fallback.

Pinning (what checks each oracle function against something independent of
it) is listed per function in the module docstrings and exercised by
tests/test_oracle.py.
"""
