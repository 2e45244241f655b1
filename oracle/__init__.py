"""CPU restatement of StreamVoxel's per-step generation hot path — TEST INFRASTRUCTURE ONLY.

This package is the oracle the tests hold the product to. Only `tests/`, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` may import it, and only to compute expected values or to time the CPU baseline.
The product package `streamvoxel_amd` never imports anything from here; on a GPU its entry points run the HIP
library or raise.

Modules (each function cites the reference file:line it restates):
  sampling.py   entropy, top_mask, block_view, block quota select (host-sync and no-sync forms), low-entropy-last
                update / quotas and the reveal schedules (numpy for the integer and ordering work, torch fp32 for the
                reference-form float reductions, numpy fp64 for the high-precision forms).
  slot.py       the low-entropy-last slot state machine (marking -> solid quota steps -> finish).
  attention.py  masked scaled-dot-product cross attention over per-slot key lengths (fp64 / fp32).
  producer.py   AxialRoPE, the cached-context window layout and the e4m3 cache quantisation.
  patches.py    the class head's patch order turned into [n, C, Y, Z, X] (explicit loops).
  backbone.py   the transformer block (LayerNorm, AdaLN modulation, GELU, rotary self-attention, MLP) in float64.
  sampler.py    the counter-based sampling tail: Philox4x64-10 uniforms per (seed, step, voxel) and the inverse
                softmax-CDF draw (float64).
The checks that pin each function (closed forms, brute force, invariants, golden vectors) are the tests named
tests/test_oracle*.py.

Parity status per function (what pins it):
  entropy_scores_f64 / entropy_scores   closed forms (uniform -> -ln C, one-hot -> 0, two-class analytic), shift
                                        invariance, fp64 vs reference-form fp32 agreement.
  top_mask                              brute force over all orderings on tiny inputs; tie-heavy cases.
  block_view / block_unview             closed-form index map, round trip.
  block_quota_select / quota_select_nosync
                                        golden vectors written by the reference (tests/golden), invariants (exactly
                                        k, subset of mask, block balance within +-1 in the fresh state, the fresh 4^3
                                        closed form).
  low_entropy_last_update               brute-force column/layer scans; golden vectors for the fp32 threshold compare.
  counts / low_entropy_last_quotas      golden vectors written by the reference; sum/positivity invariants.
  LowEntropyLastSlot                    golden trajectories written by the reference (tests/golden).
  cross_attention_f64                   brute-force per-query softmax loop on tiny inputs; padding invariance.
  producer.axial_rope / rope_frequencies golden vectors written by the reference's AxialRoPE; known answers.
  producer.window_kv / quantize_e4m3    layout and format invariants.
  patches.to_class_major                loops against torch's permute of the reference's form; the 4^3 block order.
  backbone.layer_norm / gelu / silu     invariants (zero mean, var / (var + eps)), known values (Phi(1), sigmoid(1)),
                                        odd-part identities.
  sampler.philox4x64 / uniforms         numpy.random.Philox (the same generator, one counter step apart); the
                                        uniforms' fp32 format, moments and deciles.
  sampler.invert / sample_chosen        closed forms (equal logits -> floor(u C), two-class and dominant-class
                                        rows, -inf classes), frequencies against softmax over 20 000 draws.
  backbone.rotary_attention / block     closed forms: uniform scores -> proj(mean V), one token -> proj(v), zero
                                        positions -> brute-force attention, zero gates -> identity, unit gates with a
                                        zero MLP -> x + attn + bias.
"""
