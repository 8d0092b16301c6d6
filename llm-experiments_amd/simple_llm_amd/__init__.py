"""simple_llm_amd: the KV-cache hot path of s-i-e-v-e/llm-experiments' simple-llm,
rebuilt for one MI355X (gfx950).

  gpu/        drop-in for simple-llm/src/gpu's KV-cache API over libskv.so
  _lib.py     ctypes binding of the C ABI (include/skv.h)
"""
