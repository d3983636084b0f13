"""CPU oracle for the chunkwise log-linear attention path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package
(``log-linear-attention_amd/``) may import, call or link anything in this
directory.  The only permitted users are ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py``, and they use it strictly as the
checker (or as the timed CPU baseline), never as the thing being measured or
shipped on the GPU path.

Contents (each function cites the reference file:line it restates):

* ``levels``  -- the weak Fenwick level function (recursive restatement and
  closed form ``bit_length(t ^ s)``) and the level schedule of the chunk scan.
* ``mamba2``  -- log-linear Mamba-2: materialised O(T^2) H-matrix form,
  Fenwick recurrent form, chunked form (masked chunk-level combination) and
  chunked level-scan form; plain (non-hierarchical) SSD scan for the
  lambda == 1 special case; backward through autograd; the Mamba-2 layer
  scan with its pre- and post-processing (dt softplus, x dt, A dt, lambda
  modes, D residual) on top of the chunked level-scan form.
* ``gdn``     -- log-linear Gated DeltaNet: recurrent form (matrix gates),
  materialised pair sum, chunked UT / WY form with per-level delta-rule scans,
  the plain gated delta rule (lambda == 1) and the l2norm / scale boundary.

Pinning (what checks each function against something other than itself) is
listed in each module docstring; the tests that perform the checks live in
``tests/test_oracle_*.py``.
"""
