"""TEST INFRASTRUCTURE ONLY -- the parity oracle of the MSDA path.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
may import, call, link or execute anything in this directory, and only as the
checker. The product (``muspace_amd``) never imports it and has no CPU
fallback through it.

Contents
  msda_torch.py   op-for-op restatement of the reference PyTorch path
                  multi_scale_deformable_attn_pytorch
                  (/root/reference/mu_space/ops/multi_scale_deformable_attn.py:26-58),
                  run on the CPU; forward and autograd backward. This is the
                  oracle the HIP kernels are compared with, and the timed CPU
                  baseline ("port").
  msda_direct.c   independent float64 restatement of the same operator as
  msda_direct.py  explicit loops over the closed form (bilinear sampling with
                  zero padding, x = loc_x*W - 0.5) and its analytic gradients
                  (/root/reference/csrc/ms_deformable_attn/ms_deform_attn_musa_kernel.muh:39-166);
                  used to pin msda_torch.py, not to check kernels directly.
  Makefile        builds msda_direct.c into oracle/build/libmsda_direct.so.
  msda_softmax.py the operator with its weights given as logits (softmax over
                  each query's L*P samples per head, then msda_torch); autograd
                  and a closed-form logit gradient (tests/test_oracle_softmax.py).

How each function is pinned (tests/test_oracle.py)
  * msda_torch vs msda_direct (two independent formulations) at float64;
  * the reference tests' known answers: all locations -1 -> zero output and
    zero gradients (tests/ops/test_multi_scale_deformable_attn.py:245-253),
    the width-1000 half-pixel case -> exactly 2048 (:430-468), zero queries
    (:269-280), output shapes (:95,138,160);
  * closed forms: pixel-centre sampling returns the stored value, a linear
    value field is reproduced exactly with location gradients (a*W, b*H),
    out is linear in value and in attention_weights (adjoint identities);
  * torch.autograd.gradcheck of msda_torch and finite differences of
    msda_direct;
  * planted mistakes (x/y swapped, missing -0.5, dropped corner) fail them.
The reference ships no stored golden tensors; the only fixture file
(tests/fixtures/bevformer_msda_shapes.yaml) is shape metadata, mirrored in
tests/golden/.
"""
