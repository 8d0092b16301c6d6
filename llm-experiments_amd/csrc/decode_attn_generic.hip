// Pass 1 of cached decode attention for head dims other than 64 and 128,
// contiguous caches (paged ones: decode_attn_generic_paged.hip).
//
// The reference's decode kernel takes any head_dim (a runtime loop over the
// row, simple-llm/src/gpu/gpu_kernels.py:2846, 2856-2866, 2916-2921), and the
// models its auto-configuration trains use head dims of 24 to 80
// (simple-llm/src/hyper.py:63-79). These kernels are the ones of
// decode_kernels.h with the head dim padded to DP, a power of two in
// [32, 2048]: lane i of a row of 16 lanes (DP up to 256; 128 with G = 8)
// or 64 lanes (a wavefront, past that) owns DP/16 or DP/64 consecutive
// elements, and the lanes (or parts of a lane) past the real head dim D read
// an in-row address, meet a zero query and store nothing. Loads are the
// widest vector that divides D (up to 16 bytes), or single elements.
#include "decode_kernels.h"

int skv::dec::launch_partial_generic(const DecodeArgs& a, int G, bool bf16_cache,
                                     hipStream_t s) {
  return bf16_cache ? launch_generic<uint16_t, false>(a, G, s)
                    : launch_generic<float, false>(a, G, s);
}
