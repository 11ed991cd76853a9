"""CPU oracle for the qcom_htp hot paths -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import anything from this package, and only to check or to time
the reference's CPU algorithm.  The product (``qcom_htp_amd``) never imports it:
every output the product returns comes from the HIP kernels.

Modules
-------
qmm      restatement of the reference's float-derived quantized-matmul oracle
         (``output_ref_q``) plus its integer contracts.
layouts  restatement of the reference's weight/bias carrier packers.
gdn      GDN/KDA triangular-solve oracles (fp64 inverse, forward substitution,
         the int16 block model) and the A-build of a GDN chunk.

Pinning status is recorded at the top of each module.
"""
