"""Oracle libraries for the TriTierCache HIP path (test infrastructure only).

``oracle.binding`` loads ``oracle/libtt_oracle.so`` (the C restatement of the
reference algorithm) and, where it has been built, ``oracle/_ref/libttref.so``
(the reference's own C++ sources compiled with its own flags). Only tests/,
``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg import this
package, and only as the oracle or the timed CPU side; the product package
``tritiercache_amd`` never does.
"""
