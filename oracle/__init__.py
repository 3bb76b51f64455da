"""CPU oracle for the fused dequant-matmul path — TEST INFRASTRUCTURE ONLY.

This package is a numpy restatement of the reference algorithms on the packed-weight
dequant -> GEMV/GEMM path. Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``
(its ``cpu_baseline`` leg and the output checks after each timed region) may import it,
and only to check results or as the timed CPU baseline, never as the thing measured.
The product path (``vybforge_amd`` + ``libvybdq.so``) never imports or calls anything here
and fails loudly when the HIP library is missing.

Modules and the reference code each one restates (paths relative to the reference
repository root):

  formats  q4_0 decode      HANDOFF-VYB-NATIVE-INFERENCE.md:35 (deq_q4_0 spec),
                            native/kernels/deq.vyb:4-12, native/gguf/mk_fixture.vyb:86-99,
                            native/gguf/dequant_gguf.vyb:118-127 (fixture order)
           Q8_0 decode      native/tools/q8_0_ref.py:50-56, native/kernels/q8_0.vyb:11-30
           xq8 quantizer    native/kernels/rgemv7.vyb:195-214
  exl3     mcg decode, slot map, Hadamard-128, full dequant
                            native/exl3/exl3_ref.py:31-120, native/exl3/README.md:24-49,
                            native/kernels/exl3.vyb:375-422; the f64 / f32 pipeline stages
                            exl3hgen, exl3had1, exl3had2, exl3deq32 (exl3.vyb:36-242)
  moe      route / clamped SwiGLU / combine
                            native/glm53/moe_ref.py:25-112, native/kernels/moe.vyb:1-170
  matmul   fp64 GEMV/GEMM gates and the tolerance metric
                            native/kernels/rgemv.vyb:13-15,359-366, native/tools/gen_rpf.py:2-8,
                            native/glm53/verify_layer0.py:134-139; the xq8-activation GEMV
                            gate (gemv_xq8_f64) of gemv_iq2s_q / gemv_q4k_q / gemv_q5k_q
                            (native/kernels/rgemv7.vyb:3-96, rq4kq.vyb:7-274, rq5kq.vyb:8-268)
  kquants  Q4_K / Q5_K / Q6_K decode
                            native/kernels/q4k.vyb:1-70, native/tools/q4k_ref.py:37-60,
                            native/tools/q5k_ref.py, native/gguf/q6k_verify.py:20-40
  iquants  IQ2_S decode     native/kernels/rgemv.vyb:24-80, native/tools/iq2_s_ref.py,
                            grid as native/gguf/iq2s_tables.py holds it
  producers RMSNorm / SwiGLU with the q8 copy (rms_blkg VYB_RMSQ8, silu32q VYB_SWQ8)
                            native/kernels/layer.vyb:989-1066,1551-1590, vmath.vyb:7-40

Pinning (what checks each function, all under tests/):
  q4_0 decode      the reference's frozen GGUF fixture block (interleaved order) and
                   brute force per nibble; ggml order against the public block layout
                   via an independent bit-level decoder.                 -> pinned
  Q8_0 decode      closed form d*q checked against an independent int8/fp16 bit decode
                   (no reference-held fixture exists).                   -> pinned (closed form)
  xq8              round-trip bound, RNE ties, zero block, saturation.   -> pinned (properties)
  exl3 decode      all-zero-trellis KAT (1.84375), exhaustive 65536-window check against
                   an integer-only fp16 decode, slot-map invariants.     -> pinned
  exl3 codebook    only mcg (cb 1) exists, as in the reference (exl3_ref.py:19-22);
                   any other codebook id raises ValueError.              -> pinned (KAT above)
  exl3 dequant     closed form of the all-zero trellis after the Hadamard sandwich,
                   H orthogonality, per-block linearity.                 -> pinned
  exl3 stages      map_deq equals the pinned map decode; hgen equals the scaled Sylvester
                   matrix; had1 equals the pinned column transform; had2 after had1 equals
                   the pinned block rotation.                            -> pinned
  moe              the reference's committed MoE goldens (routing ids/weights, and the
                   block output on a column slice).                      -> pinned
  matmul           fp64 numpy matmul (invariant).                        -> pinned
  gemv_xq8_f64     against the reference kernels' factored integer form
                   (sum_b dw*dx*sum q_w q_x) and against the exact GEMV when x
                   quantizes losslessly.                                 -> pinned
  kquants          blocks assembled byte by byte from the layout description
                   against closed-form per-element values; scale/min packing round
                   trip; Q5_K without high bits = Q4_K; Q6_K exact in float32
                   (tests/test_kquant_oracle.py).                        -> pinned
  iquants          grid structure (magnitudes in {8, 25, 43}) and byte-assembled
                   IQ2_S blocks against closed-form values
                   (tests/test_iquant_oracle.py).                        -> pinned
  producers        seeded Newton sqrt against the reference's 24-step loop and the
                   correctly rounded sqrt; ordered sums against exact integer and
                   rational sums; the reference's exp within its stated 1e-9 of libm;
                   RMSNorm closed form; the q8 copy is xq8
                   (tests/test_producers_oracle.py).                     -> pinned
Every function above is pinned; none is "parity unpinned".
"""
