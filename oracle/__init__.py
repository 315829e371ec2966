"""CPU oracle for flash-spacetime attention -- TEST INFRASTRUCTURE ONLY.

This package restates the reference specification
(`src/flash_spacetime/reference.py` of sevmag/flash-spacetime) on the CPU,
generalised from the reference's `W [C, C], C == D` to the nn.Linear layout
`W [D, C]`, plus a chunked float64 evaluator of the forward and of the exact
backward for shapes whose materialised pair tensor would not fit in memory.

It exists to CHECK the HIP implementation. Only `tests/`,
`__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may
import it; the product package `flash_spacetime_amd` never does, and its
operators fail loudly when the HIP library is missing instead of falling
back to anything here.

How each function is pinned (tests/test_oracle.py):
  * constants and the frequency ladder: closed forms and the golden vectors
    generated from the reference in `tests/golden/`;
  * pair angle / embedding: closed forms (diagonal, saturation, symmetry,
    sign(0) = 0) and a scalar pure-Python brute force;
  * eager attention: golden vectors from the reference (fp64, fp32, bf16,
    C == D), a scalar brute force, flags-off == scaled_dot_product_attention,
    the L = 1 closed form, bias-shift invariance;
  * chunked fp64 forward/backward: equality with autograd through the eager
    restatement, `torch.autograd.gradcheck`, and the closed forms
    (L = 1 gradients, db, rowsum(dS) = 0);
  * the row-block evaluator `event_rows_fp64`: its blocks summed over an
    event equal the chunked whole-event evaluators, and a block's gradients
    equal those of the whole event with the upstream gradient zeroed
    outside the block.
"""

from .spec import (  # noqa: F401
    SINEMB_CLIP,
    SINEMB_INPUT_SCALE,
    SINEMB_N_FREQ,
    TIME_SCALE,
    attention,
    attention_fp64_chunked,
    backward_fp64_chunked,
    event_rows_fp64,
    float_padding_mask,
    frequencies,
    pair_angle,
    pair_angle_rect,
    embed_angle,
    pair_embedding,
    pair_features,
    pair_mask,
    valid_row_mask,
)
