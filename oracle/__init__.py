"""CPU oracle for WhiteMatter's attention hot path - TEST INFRASTRUCTURE ONLY.

A restatement of the reference's portable algorithm (Cy-47/White-Matter,
src/white_matter/ops/) used to check the gfx950 kernels and the host code:

  oracle.metadata   numpy restatements of the three metadata builders
  oracle.attention  float64 explicit-softmax attention under the reference's masks
  oracle.kv_pool    the KV-pool key norm, RoPE and pool write with the
                    reference's rounding points

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker or the timed CPU baseline; the
product (white_matter_amd) never imports or calls it.

Pinning (each function is checked against more than its own formula):
  - cyclic metadata: known answer of tests/unit/test_ops.py:77-86 and
    brute-force counting of ids (tests/test_oracle.py);
  - feedback metadata: exact equality with the cyclic builder
    (tests/unit/test_metadata.py:10-23) and brute-force run scans;
  - strict metadata: known answers tests/unit/test_jacobi_flash_packing.py:15-16
    and tests/unit/test_strict_causal_attention.py:177-180, golden vectors
    where present (tests/golden/), structural invariants and end-to-end
    equality of attention through the schedule with a per-query loop that
    never builds a schedule (tests/unit/test_strict_causal_attention.py:16-39);
  - attention: PyTorch's math SDPA (the reference's own call), a per-query
    loop, equal-score and exact-zero invariants, float64 at 1e-12;
  - kv_pool: the same steps written with PyTorch's F.rms_norm and tensor ops
    in the key dtype on the CPU, and RoPE rotation invariants.
"""
