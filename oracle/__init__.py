"""Oracle for the GPU KV-partition path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
anything from this package, and only to compare results against (or, for
bench.py, as the timed CPU baseline).  The product (scope_amd) never imports it.

Contents
  attn_np.py        numpy restatement of the reference's decode-attention math:
                    fp64 closed forms (the mathematical pin), an fp32 blocked
                    online softmax with tile merge, the pairwise LSE merge, the
                    reference triple conventions, and the partition / page /
                    boundary integer model.
  cpu_attn_port.c   C restatement of the reference CPU partial kernels
                    (kernel/cpu_attn.cpp: fused_cpu_attn, fused_cpu_attn_mla,
                    fused_cpu_attn_mla_compressed) with OpenMP, used to verify
                    results at full sizes; bench.py times it beside the CPU
                    baseline (the clean-room host kernel) as context.
  port.py           ctypes binding of the C restatement.
  Makefile          builds oracle/_build/libwsoracle.so with gcc.

The reference CPU kernel itself is not built here, and oracle/_ref stays
empty.  The reason is its licence, not the toolchain: the reference README
(README.md:60-62) reserves all rights and forbids derivative works, and using
the reference as a running oracle was made conditional on an owner's
confirmation that this pipeline has no channel to obtain.  (Technically
kernel/cpu_attn.cpp would build through torch.utils.cpp_extension against
libtorch and pybind11, kernel/build.py:13-25, both present in the image.)
"""
