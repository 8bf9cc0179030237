"""CPU oracle of the fused attention family -- TEST INFRASTRUCTURE ONLY.

Used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as
the checker; never imported by the product package.

  naive.py   fp32 torch restatement of reference_implementations.py:11-52
             plus the benchmark harness's side-product formulas
  brute.py   fp64 explicit-loop attention that pins naive.py on tiny inputs
  inputs.py  seeded input generation shared by tests and bench

Pinning (every function below is checked by tests/test_oracle.py):
  - naive.reference_forward vs brute.brute_forward on tiny shapes (MHA,
    GQA, causal top-left / bottom-right, M < N, M > N, empty rows, split);
  - committed fixtures tests/golden/*.npz written by tests/golden/make_fixtures.py
    from brute.py;
  - closed forms: constant keys -> uniform softmax weights; softmax rows sum
    to 1; sum of softmax column sums = group size x non-empty rows;
    sum(row_sum) = sum(col_sum); GQA = MHA with repeated K/V; split = M
    gives zero cross sums;
  - naive.naive_attention_with_scores vs reference_forward (top-left offset);
  - mutation tests: planted mistakes in the oracle fail the pins.
"""
