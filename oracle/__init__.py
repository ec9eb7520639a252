"""CPU oracle for history-only PCP attention.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` may import this package, and only as
the checker (or, for ``bench.py``, as the timed CPU baseline).  The product
(``aws_training_study_amd``) never imports it and has no CPU fallback.

``oracle.pcp_oracle`` restates the Trainium2 proof of concept's executable
specification (pcp_attention/config.py, layout.py, reference.py,
kernel.py:17-29, run_poc.py:81-169) in numpy (index maps, float64 attention)
and, for the ring model that is also the timed CPU baseline, in torch FP32
with the reference's loop order.
"""
