"""CPU oracle for the geometric-attention hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import anything from this package, and only as the checker or
the timed CPU baseline.  The product (``matterformer_amd``) never imports it:
its ops run on the HIP library or raise.

Contents:
  simplicial.py  torch-CPU restatement of the reference's 2-simplicial torch
                 path (its execution shape: padded, chunked, masked_fill with
                 finfo.min) + an independent float64 numpy brute force.
  knn.c/knn.py   brute-force kNN with the stable (d^2, j) order (C, no FMA).
  radius.c/radius.py
                 27-image minimum-image radius mask (C, no FMA) + a float64
                 dense masked-softmax attention.

Pinning (what each function is checked against) is listed in the header of
each module.
"""
