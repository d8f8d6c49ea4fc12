"""CPU oracle for the QStore hot path -- TEST INFRASTRUCTURE ONLY.

A from-scratch numpy restatement of the reference (JHollenb/mrun-pub) algorithms on the
quantized-weight path; every function cites the reference file:line it follows.  Only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this package, and only as the checker / the timed CPU baseline.  The product package
(``mrun-pub_amd/``) never imports it and has no CPU fallback.

Pinning (what checks each function against something other than its own formula) is listed
in each module's docstring; a function with no such check is marked "parity unpinned".
"""
