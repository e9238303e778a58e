"""CPU oracle for the KDA mixer hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package, and only as the reference the
HIP results are compared with or as the timed CPU baseline, never as the
thing measured or shipped.  The product
package ``sophia_amd`` does not import it and has no CPU fallback.

* ``kda_oracle`` -- numpy restatement of the reference's CPU path
  (ml/runtime/model/attention.py:17-60, 226-294, 373-420).
* ``kda_ref.c``  -- the same per-token recurrence in C (OpenMP over
  sequence x head), built by ``oracle.build`` into ``oracle/_lib``.
* ``c_oracle``   -- ctypes binding of ``kda_ref.c``.

The reference's own Python cannot be imported here (it needs Python >= 3.12
syntax and the external flash-linear-attention package), so ``oracle/_ref``
is not built; the restatement is pinned by closed forms and invariants.
"""
