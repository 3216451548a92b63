"""Oracle for the fused causal attention path -- TEST INFRASTRUCTURE ONLY.

CPU restatement of the reference's algorithm, used as the checker by tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg.  Nothing in the product
(fused-attention_amd/) imports, links or runs anything from this package.

Modules
  attention_oracle  numpy float64 restatement: forward (MHA/GQA), LSE, Delta,
                    closed-form gradients, row-sampled evaluation, the tiled
                    online-softmax algorithm, and a pure-Python loop version
  cases             the reference's seeded correctness-case generators
  cpu_reference     the reference's PyTorch fp32 path (chunked), timed as the CPU baseline

Parity pinning (every function is checked by tests/test_oracle.py against
something other than a retyped formula):
  forward           pure-Python loops on tiny inputs; torch SDPA (float64, a library
                    routine); row 0 == V[0]; Q = 0 gives prefix means of V;
                    tiled online softmax == closed form for every tile pair
  GQA               equals MHA on explicitly repeated K/V; H_kv == H reduces to MHA
  LSE               scipy.special.logsumexp of the masked scores; rows of
                    exp2(s*c - lse) sum to 1
  Delta             rowsum(dO*O) == rowsum(P*dP) (independent identity)
  gradients         central finite differences (float64, tiny inputs) and torch
                    autograd of SDPA in float64
  row sampling      equals the full evaluation on the sampled rows
  cases             seeds are crc32 of the case id; count and order of the
                    reference's lists (84 / 96 / 7); planted-mistake tests show
                    the checks fail for a wrong sign, a dropped scale or a
                    transposed operand
cpu_reference (tests/test_cpu_reference.py) is pinned against the float64 oracle above:
  explicit formula  MHA, GQA and MQA shapes, plus row 0 == V[0] and the prefix means of Q = 0
  head chunking     budgets that split the heads into ragged chunks and whole GQA groups
                    (g = 1, 2, 4, 8), equal to one unchunked pass; mutated copies (wrong
                    K/V head index, chunks straddling a group, the last K/V head rounded
                    down, a shifted output slice) are caught
  fp32 autograd     dQ, dK, dV for MHA and GQA (group sums), the single 1/sqrt(D) factor
No function is left "parity unpinned".
"""
