"""CPU oracle for the PopKV retrieval path (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
may import this package, and only as the checker.  The product package
(``popkv_amd``) never imports it.

* ``oracle.core``     -- ctypes front end of ``popkv_oracle.c``: the bit-exact
  restatement of the reference's production arithmetic.
* ``oracle.readable`` -- numpy restatement of the reference's readable
  (dense-reconstruction) references, used to pin the core within the
  reference's own tolerances.
"""
from . import core, readable  # noqa: F401
