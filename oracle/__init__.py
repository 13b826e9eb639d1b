"""CPU oracle of the attention hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the semantics of the reference's hot-path
ops (paths relative to the reference checkout; each function cites the lines
it follows).  Floating-point ops run in torch fp32 (or fp64) on the CPU;
integer/index work (slot mapping, block allocation, the KV scatter) runs in
numpy or plain Python.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import it, and only as the checker or the timed CPU baseline -- never as the
product path.  The product ops (mycustomcudaengine_amd.ops) have no CPU
fallback.

How each function is pinned (tests/test_oracle.py):
  decode_attention_ref   torch SDPA (enable_gqa) on the gathered KV, a scalar
                         brute force on tiny inputs, block-table permutation
                         invariance, NaN-sentinel pool, ctx == 1 -> v_0.
  prefill_attention_ref  causal torch SDPA (enable_gqa), scalar brute force,
                         S == 1 -> v_0, row 0 -> v_0.
  rmsnorm_ref            torch.nn.functional.rms_norm, scalar brute force.
  rope_tables/rope_ref   complex-exponential rotation, pos 0 == identity,
                         per-pair norm preservation, composition of angles.
  swiglu_ref             torch.nn.functional.silu, math.exp brute force.
  kv_store_ref           scalar Python loop; slot < 0 skipped.
  BlockAllocatorRef      hand-enumerated FIFO sequences.
  slot_mapping_ref       brute force over the allocator's tables.
  decode_advance_ref     the allocator's slot_of() on the positions it yields,
                         -1 past the table width (hand-built cases).
  argmax_rows_ref        numpy.argmax; torch.argmax on ties and NaN rows.
  prefill_paged_ref      the last S rows of prefill_attention_ref over the
                         whole sequence (cached prefix + chunk).
  LlamaRef (model_ref)   tests/test_model_oracle.py: with every projection
                         weight zero the layers are the identity, so logits
                         equal rms_norm(embed[ids]) @ embed^T; an independent
                         forward built from library routines (F.rms_norm,
                         causal SDPA with enable_gqa, F.silu, complex-
                         exponential RoPE) on non-unit norm weights, for
                         prefill and prefill + decode; each of nine planted
                         mistakes in that forward (a dropped residual, gate
                         and up swapped, RoPE on v or missing on k, norms
                         swapped or unweighted, a wrong GQA map, no causal
                         mask, a shifted position) must move the logits far
                         outside the tolerance.  Also prefill(S) ==
                         prefill(S - 1) + decode (tests/test_engine_cpu.py).
"""
