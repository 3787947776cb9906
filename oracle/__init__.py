"""CPU oracle for the SunShape compressed-KV attention path.

TEST INFRASTRUCTURE ONLY.  This package is a from-scratch CPU restatement of
the reference's arithmetic (gauravsaini/sunshape-mlx) used as the checker for
the HIP path.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it.  The product package never
imports, links or executes anything from here: when the HIP library is
missing, the product raises instead of falling back to this code.

Modules
-------
``sunshape_oracle``  NumPy restatement (float64 arithmetic where the
                     reference's result is defined up to rounding).
``encode_ref.c``     Plain-C float64 brute-force block-VQ encoder (same
                     contract as ``sunshape_oracle.encode_blockvq``), compiled
                     by ``oracle/build_oracle.py`` into ``oracle/_build/``.

Pinning status of every function is listed in ``sunshape_oracle.__doc__``.
"""
