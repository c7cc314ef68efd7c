"""CPU oracle for the dtmi backward / gradient / optimizer path.

TEST INFRASTRUCTURE ONLY. This package is a NumPy restatement of dtrain's
arithmetic (siddhaantxsingh/DISTRIBUTED-TRAINING, pure Python over NumPy); each
function cites the dtrain file:line it follows and performs the same NumPy
operations in the same order with the same dtype promotion (NumPy 2 rules), so
that on identical inputs it produces what dtrain produces. Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg import it, and only as
the reference results to compare against or the timed CPU baseline -- never as part of the product path
(the dtmi package never imports it).

Pinning (what stops a plausible mistake here from going unnoticed):
  ops.py      finite differences (dtrain's own check() recipe), closed forms,
              brute-force loops on tiny inputs, torch float64 autograd, and the
              golden vectors written from dtrain itself (tests/golden/).
  model.py    golden vectors from dtrain (init draw order, one full step in
              float64 and float32), finite differences of the loss.
  optim.py    golden vectors from dtrain (float32 weak-scalar rounding),
              torch.optim.AdamW agreement, bit-exact float64 restatement.
  ddp.py / zero.py / comm.py
              closed forms (fixed-order sum), invariants (bucket size and
              grouping do not change results, ZeRO shard == full AdamW slice,
              state bytes == 2*itemsize*ceil(n/W)).
"""
