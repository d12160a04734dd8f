"""CPU oracle for the MoE FFN hot path — TEST INFRASTRUCTURE ONLY.

This package is the checker: a C++ restatement of kestrel's AVX2 CPU path
(crates/kestrel-engine/src/{quant,qdot,avx2,transformer}.rs) built into
``oracle/libkmoe_oracle.so``. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only to check or time
the reference arithmetic. The product library never routes through it.

Parity status of each function is listed in ``kmoe_oracle.h``; glibc ``expf``
(route softmax, SwiGLU) is "parity unpinned" by any reference test.
"""
