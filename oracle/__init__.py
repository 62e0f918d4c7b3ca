"""CPU oracle for the GPU hot-expert MoE path. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import,
call, link or run anything in this directory, and only to check results against (or, for
cpu_moe.c, as the timed CPU baseline). The product path (kt-prefill-lend_amd/)
never imports it and fails loudly when its HIP library is missing.

Contents
  gguf_ref.py   numpy restatement of the reference's GGUF block formats, its
                q8_1 activation quantizer, its int8 vec_dot sums, the window
                GEMV contract, SiLU*mul, the weighted top-k combine, the hot
                cache route lookup, a stable sort of routes by slot and the
                `_reference_check` FFN.
  cpu_moe.c     C restatement of kt-kernel's LLAMAFILE `forward_many` (the
                reference's CPU expert path), threaded; the CPU baseline.
  Makefile      builds cpu_moe.c into oracle/_build/libktoracle.so.

How each function is pinned (closed forms, invariants, brute force, known
answers) is listed in the header of gguf_ref.py. Functions with no such check
say "parity unpinned" there.
"""
