"""Parity oracle -- TEST INFRASTRUCTURE ONLY.

CPU restatement of the arithmetic of GhostSuite's per-sample-gradient samplers
(/root/reference/ghostEngines/..., cited per function in ``ghost_ref``), used as the checker
for the HIP kernels.  Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import it; the product (``ghostsuite_amd``) never does, and has no
CPU path of its own.

Modules
  ghost_ref   the reference op sequences (bf16 casts and rounding points kept) and the same
              formulas in exact arithmetic (fp64, casts removed), plus train-gradient
              formulas and the GradProj projection.
  brute       textbook per-sample gradients (one backward per sample) used to pin
              ``ghost_ref`` independently of its own formulas.

Pinning (how each oracle function is checked; see tests/test_oracle.py):
  - brute-force per-sample gradients on small models (definition of every dot product,
    train gradient and projection);
  - closed forms / invariants (pairwise == <G_i, sum_j G_j>_F; presum == pairwise when
    n_val == 1; homogeneity; Kronecker identity; embedding mask x Gram);
  - known answers from reading the reference (choose_ki_ko on GPT-2 shapes, the 2T^2 rule
    on the BASELINE shapes);
  - golden vectors written by the reference's own functions (tests/golden/make_golden.py,
    run in the build container only; tests/golden/reference_vectors.pt holds inputs and
    outputs): the *_ref op sequences reproduce them bit for bit, which pins every bf16
    rounding point, and the exact forms sit within the bf16 tolerance.
The reference itself is pure Python with no compiled part: oracle/_ref has nothing to
build.
"""
