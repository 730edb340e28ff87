// prefill_attention_short: the grouped-head prefill attention kernel with
// 16-query workgroups, for sequences short enough that the 32-query grid
// leaves CUs without a second workgroup (prefill_attention.hip picks it).
// A translation unit of its own so that the two sets of instantiations
// compile in parallel.
#include "prefill_v2.hpp"

namespace slc_prefill {

template <typename T, int G, int MK, bool CAUSAL>
int launch_v2_short(const void* q, const void* k, const void* v, const void* mask, void* out,
                    int64_t batch, int tokens, int kv_heads, const int64_t* st, float scale,
                    bool exact, const unsigned char* classes, hipStream_t stream) {
  return launch_v2<T, G, MK, CAUSAL, 1>(q, k, v, mask, out, batch, tokens, kv_heads, st, scale,
                                        exact, classes, stream);
}

#define SLC_SHORT_ONE(T, G, MK, C)                                                                \
  template int launch_v2_short<T, G, MK, C>(const void*, const void*, const void*, const void*,  \
                                            void*, int64_t, int, int, const int64_t*, float, bool, \
                                            const unsigned char*, hipStream_t);
#define SLC_SHORT_MK(T, G, MK) SLC_SHORT_ONE(T, G, MK, true) SLC_SHORT_ONE(T, G, MK, false)
#define SLC_SHORT_G(T, G)                                                                  \
  SLC_SHORT_MK(T, G, 0) SLC_SHORT_MK(T, G, SLC_BF16 + 1) SLC_SHORT_MK(T, G, SLC_F16 + 1) \
  SLC_SHORT_MK(T, G, SLC_F32 + 1)
#define SLC_SHORT_T(T) \
  SLC_SHORT_G(T, 1) SLC_SHORT_G(T, 2) SLC_SHORT_G(T, 4) SLC_SHORT_G(T, 7) SLC_SHORT_G(T, 8)
SLC_SHORT_T(slc::bf16_t)
SLC_SHORT_T(slc::f16_t)
#undef SLC_SHORT_T
#undef SLC_SHORT_G
#undef SLC_SHORT_MK
#undef SLC_SHORT_ONE

}  // namespace slc_prefill
