"""CPU oracle for representax's quantized-linear path.

TEST INFRASTRUCTURE ONLY. This package restates, in numpy with bit-level
codecs, the numerics of

* ``src/representax/models/adapters.py:30-79,141-182`` (bf16 bit casts, the
  per-output-row INT4 packer and unpacker, the INT4-LoRA forward and its JAX
  autodiff transpose), and
* ``src/representax/precision.py:127-239`` (dynamic amax scaling, OCP fp8
  casts, the scaled fp8 dot and its custom VJP),
* ``src/representax/models/components.py:153-167``,
  ``bert/model.py:243-249`` and ``qwen3_vl/text.py:200-203`` (the GELU and
  SiLU-gated FFN steps next to the linears, ``act``),
* ``src/representax/tasks/retrieval/mnr.py:48-52,132-158,338-341`` (the
  in-batch multiple-negatives ranking loss of the train-step harnesses,
  ``mnr``),

so that tests, the smoke check and the benchmark's CPU-baseline leg can check
the HIP kernels of ``representax_amd``. Nothing in the product imports it; the
product fails loudly when its HIP library is missing instead of falling back
here.

Pinning (what checks each function against something other than itself):

* ``codecs``: bf16 and fp8 casts are compared with torch's own
  ``bfloat16``/``float8_e4m3fn``/``float8_e5m2`` conversions (a library
  routine) over every bf16 bit pattern, every fp8 code, and boundary sweeps;
  the decoders are compared with the OCP fp8 closed form.
* ``int4``: hand-built known answers (zero rows, ties-to-even, clipping,
  odd K padding, nibble order), exhaustive unpack over all 256 byte values,
  and the pack/unpack round-trip bound.
* ``lora``: forward compared with the merged-weight closed form and an fp64
  brute-force loop on tiny shapes; backward compared with central finite
  differences of the fp64 forward and with closed-form identities.
* ``fp8``: amax/scale closed forms (zero, inf, NaN tensors), cast through the
  torch-pinned codec, dot compared with an fp64 product of the exactly decoded
  operands, VJP compared with the transposed-product identities.
* ``mnr``: brute-force loops, the orthonormal closed form
  (log(e^s + n - 1) - s per row, a zero row clamped at 1e-12), torch's
  float64 logsumexp and autograd, and central finite differences on exactly
  representable steps.
* ``act``: GELU and SiLU against torch's float64 routines and closed forms
  (gelu(0) = 0, gelu(-z) = gelu(z) - z, silu(-g) = silu(g) - g), their
  derivatives against central finite differences, the fused blocks' backward
  against finite differences of their float64 forward.

Parity unpinned (no reference test or fixture fixes these bits, and the
reference cannot run here): XLA:CPU's accumulation order of bf16 dots, whether
its f32->f8 convert rounds directly or through f16, and whether bf16-typed
elementwise ops keep excess precision. The oracle takes the HLO-typed reading:
every bf16-typed op rounds once to nearest-even and f32->f8 rounds directly.
The FFN activations (``act``) are the exception: evaluated exactly from the
bf16 linear outputs and rounded once, the fused-elementwise reading.
"""
