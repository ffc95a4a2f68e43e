// Head-dim 384 forward (attn_fwd_d384.hip), reached through aa_attn_fwd /
// aa_attn_fwd_workspace / aa_attn_fwd_noalloc when args->hd == 384.
#pragma once

#include "aa_common.h"

namespace aa {

// Most bytes of split partials the d=384 forward needs on a 256-CU device
// (256 key ranges x 128 queries x (384 bf16 + 1 float)).
constexpr size_t kD384MaxPartialBytes = (size_t)256 * 128 * (384 * 2 + 4);

// Bytes of split partials the d=384 forward needs on a device with ncu CUs.
size_t attn_fwd_d384_workspace(int64_t B, int64_t Sq, int64_t Sk, int64_t H, int ncu);

// Validates `a` (hd == 384, bf16) and launches the forward (plus its combine
// pass when the keys are split); AA_* code.
int attn_fwd_d384(const aa_attn_fwd_args* a, int ncu, hipStream_t stream);

}  // namespace aa
