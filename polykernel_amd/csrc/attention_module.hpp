// attention_module.hpp -- the entry points of an emitted attention code
// object, handed to the attention dispatcher (attention.hip) by the runtime's
// code-object launcher (csrc/runtime/launchers.cpp).  Host-only.
#pragma once

#include <cstdint>

#include "../../include/polykernel_amd.h"

namespace pk {

// hipFunction_t handles (as void *) of one emitted object, launched instead of
// the linked kernels.  A flash-kernel config (D 64 / 128) has fa_fused and
// fa_combine; the generic config has att, att_unaligned, att_combine and
// kv_append.  Null entries are errors only if the dispatch needs them.
struct AttModule {
  void *fa_fused = nullptr;
  void *fa_combine = nullptr;
  void *att = nullptr;
  void *att_unaligned = nullptr;
  void *att_combine = nullptr;
  void *kv_append = nullptr;
};

// pk_fused_kv_append_attention_config with the kernels of `mod` (null: the
// linked kernels): the same tile-shape, key-split, workspace and append
// decisions either way, so an emitted object gives the linked kernels' bits.
int fused_kv_append_attention_module(const uint16_t *Q, uint16_t *Kc, uint16_t *Vc, const uint16_t *Kn,
                                     const uint16_t *Vn, uint16_t *O, int B, int H, int S_q, int S_cache, int D,
                                     int cache_capacity, float scale, int causal, const pk_config *cfg,
                                     const AttModule *mod, void *stream);

}  // namespace pk
