"""Test infrastructure only: the CPU oracle for the GMM EM hot path.

Nothing in the product package (``gmmxx_amd``) imports this package.  Only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker.
"""
