"""CPU oracle for DCR-Attention's sparse decode path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
checker.  The product package (``dcr_attention_amd``) never imports it.

Modules
-------
``cpu``        ctypes wrapper over the C restatement ``dcr_oracle.c``.
``torch_twin`` the reference's M1 oracle restated with the same torch calls
               (qaxis_topk_reference.py:42-259), used to pin ``cpu``.
"""
