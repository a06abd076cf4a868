"""CPU oracle for the nine-op suite -- TEST INFRASTRUCTURE ONLY.

Nothing in the product (autokernel_amd/) imports this package. Only tests/, the smoke check in
__graft_entry__.smoke() and the cpu_baseline leg of bench.py may use it, and only as the checker
or as the timed CPU baseline -- never as a result the product returns.

  reference_ops  restatement of the reference's reference.py on PyTorch CPU: the same sequence
                 of tensor ops, so f16 / bf16 intermediate rounding matches the reference.
  brute          independent numpy float64 (and float16-emulating) restatements used to pin
                 reference_ops; no torch.
  inputs         the seeded input generators of the reference's bench.py and BASELINE configs,
                 generated on the CPU so host and GPU see identical bits.

Pinning (every function of reference_ops has at least one):
  * golden fixtures under tests/golden/ written by numpy brute force (make_golden.py);
  * fp64 brute force on small random inputs;
  * closed forms (softmax rows sum to 1, constant rows, identity / quarter-turn rotations,
    log(V) cross entropy, identity matmul, causal row 0 = V[0], zero up-projection, ...);
  * the reference harness's adversarial-input rules (overflow to inf in f16 and NaN rows).
"""
