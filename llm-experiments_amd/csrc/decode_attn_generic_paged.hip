// Pass 1 of cached decode attention for head dims other than 64 and 128 over
// a paged cache (the masked kernels of decode_kernels.h; contiguous caches:
// decode_attn_generic.hip). A translation unit of its own, so that the two
// kernel sets compile in parallel.
#include "decode_kernels.h"

int skv::dec::launch_partial_generic_paged(const DecodeArgs& a, int G, bool bf16_cache,
                                           hipStream_t s) {
  return bf16_cache ? launch_generic<uint16_t, true>(a, G, s)
                    : launch_generic<float, true>(a, G, s);
}
