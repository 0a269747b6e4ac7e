"""CPU oracle for the MLA decode path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import this package, and only as the checker / the timed CPU baseline.  The product path
(``mlc_decode_amd``, ``mla_decode.py``, ``baseline_mla.py``) never imports it.

Parity status of each function is stated in its module docstring.
"""
