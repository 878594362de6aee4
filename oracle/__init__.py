"""CPU oracle for the low-rank KV restore / fit path -- TEST INFRASTRUCTURE ONLY.

A numpy restatement of the reference algorithm (Tianyu9748/ReelCache,
``reelcache/restore_kernels.py``, ``reelcache/_hevc.py``,
``reelcache/node_packets.py``, ``reelcache/factorization.py``,
``reelcache/gpu_fitting.py``, ``reelcache/rank_method.py``), each function
citing the file:line it follows.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker (or the timed CPU
baseline), never as the measured or shipped path.  The product package
``reelcache_amd`` never imports it.

How each function is pinned (tests/test_oracle_*.py):
* quantize: the reference tests' known answers (tests/test_codecs.py:382-440,
  tests/test_step6_node_packets.py:73-90), the covering invariant, and
  brute-force minimality of the FP32 scale on small inputs;
* restore: closed forms (complex multiplication of pairs, float64 products
  against exact rational arithmetic), layout equivalences and the reference's
  own FP64 ``explicit_values`` restatement (tests/test_restore_kernels.py:296-303);
* fit: numpy.linalg.eigh / svd subspaces, closed-form crossings, orthogonality.
No function here is "parity unpinned".
"""
