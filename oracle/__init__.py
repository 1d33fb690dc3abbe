"""CPU oracle for the RAM-Net operator path -- TEST INFRASTRUCTURE ONLY.

A restatement of the reference's pure-PyTorch algorithm
(packages/ramnet-ops/src/ramnet_ops/impl/torch_impl.py) and an fp64 event
loop used to check the HIP kernels. Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may
import it, and only as the checker or the timed CPU baseline; the product
package (``ram-net_amd/ramnet_ops``) never imports it.

Pinning: every function is checked in ``tests/test_oracle.py`` against the
reference tests' known-answer fixtures (``tests/golden/``), closed forms of
the mathematics, fp64 brute force, and against each other (dense torch
algorithm vs sparse fp64 event loop). See ``ram_oracle.py``'s header for the
function-by-function list.
"""
from .ram_oracle import *  # noqa: F401,F403
