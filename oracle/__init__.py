"""TEST INFRASTRUCTURE ONLY -- the CPU checker for libinferbit_amd.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only to check or time the CPU
reference; the product path (``libinferbit_amd``) never imports it.

* ``oracle.pyoracle``  -- ctypes bindings of ``ib_oracle.c`` (this repo's C
  restatement of the reference algorithms) built into ``oracle/_lib``.
* ``oracle.refbind``   -- ctypes bindings of ``oracle/_ref/libinferbit_ref.so``,
  the reference library compiled from its own sources by ``oracle/Makefile``
  (used to write golden vectors and to cross-check the restatement).
"""
