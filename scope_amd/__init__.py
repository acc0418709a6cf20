"""scope_amd — MI355X (gfx950) GPU partition of a physically partitioned
decode KV cache: paged bf16 HBM store, append, split-KV GQA / absorbed-MLA
decode attention returning (out, lse), and the LSE merge with the host partial.

Modules
  ops            ctypes operator layer over lib/libwsgpu.so (include/wsgpu.h)
  cache          paged HBM partitions and host+GPU partitioned caches
  partition      boundary / share / page arithmetic (host integers)
  decode         partitioned decode step (GPU partial || host partial -> merge)
  reference_api  the reference's GPU helper signatures on the new kernels
"""
__version__ = "0.1.0"
