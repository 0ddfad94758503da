"""CPU oracle for the switched-LoRA path -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy (float64 arithmetic with explicit bf16
rounding where the reference rounds), the reference algorithm of Granite
Switch's per-token switched-LoRA path.  Each function cites the reference
file:line it follows.  It exists to CHECK the HIP implementation:

  * only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg
    of ``bench.py`` may import it;
  * the product package (``granite-switch_amd/``) never imports, calls or
    falls back to anything here.

Pinning (what each function is checked against, in ``tests/test_oracle.py``):

  mapping.promote_rank            reference KAT table (tests/unit/test_promote_rank.py:16-52)
  mapping.latest_wins             reference KATs (tests/shared/multi_switch_cases.py:66-160,
                                  tests/vllm/test_multi_switch_serving.py:168-243)
  mapping.alora_effective_ids     reduces to latest_wins with one control token at the
                                  activation offset (checked token-by-token)
  mapping.build_remap / finalize_tables
                                  hand-derived KATs (non-applicable -> 0, stable rank sort,
                                  slice_col_r / tile_to_slice numbers)
  mapping.compute_bitmasks        hand-derived KATs for the reference's 64-token pattern at
                                  BLOCK_M in {1,8,16,32,64}, sign-bit case
  mapping.build_segments          brute-force invariants (permutation, stability, counts)
  mapping.applicability           hand cases: a nonzero row past the rank does not count,
                                  one nonzero slice is enough, rank 0 never applies
  mapping.build_adapter_kind_lut / split_adapter_indices
                                  reference KATs (tests/unit/test_probe_routing.py:36-72)
  lora.switched_lora_apply        identity-weight closed form (tests/shared/lora_cases.py:355-426)
                                  and a per-token explicit loop (independent formulation)
  lora.per_token_reference        the explicit loop above; also checked against the identity
                                  closed form
  lora.shrink_rows                identity-weight closed form (z = 0.1 (a+1) x[:, :r])
  lora.switch_lora_expand_xext    equals base + switched-LoRA delta through build_w_ext
  lora.shrink_expand_xext         per-token loop over hand-packed tiers
                                  (tests/unit/test_wcross_shrink_kernel.py:41-101), base rows
                                  exactly zero, all-base tile exactly zero
  lora.expand_swiglu_xext         silu(g)*u closed form on hand values
  baseline.hf_loop                equals lora.switched_lora_apply in float64 (to 1e-12) and
                                  its "hf" rounding mode in bf16 / fp32; timed as the CPU
                                  baseline
"""
