// Paged attention for head sizes other than 128: launchers of the kernels in
// any_head.hip, called by pa_prefill and pa_decode when head_dim != 128.
#pragma once

#include <hip/hip_runtime.h>

namespace pa {

struct PrefillParams;
struct DecodeParams;

// True for the head sizes the kernels of any_head.hip are built for: the
// multiples of 16 from 16 to 256 other than 128 (the tuned kernels' size).
bool any_head_dim(int head_dim);

// Zero pass and prefill of `p` (filled as for the tuned kernel; the work
// list and pools are not used) with `head_dim`-wide rows.  Returns a PA_*
// code.
int prefill_any_launch(const char* name, const PrefillParams& p, int head_dim, hipStream_t s);

// Split kernel and merge of `p` (filled as for the tuned kernel, with
// head_dim-wide partials in the workspace and, optionally, the decode work
// list of pa_decode in p.plan) with `head_dim`-wide rows: the head sizes of
// any_head_dim, and 128 (which pa_decode sends here for bf16 pages with more
// than 16 q heads per kv head).  `code` < 0: bf16 pages; else the pages hold 1-byte codes of that
// type (kCodeE4M3, kCodeI8, kCodeU8) with per-token scales, as p.k8 / p.v8 /
// p.k_scales / p.v_scales give them.  Returns a PA_* code.
int decode_any_launch(const char* name, const DecodeParams& p, int head_dim, hipStream_t s, int code = -1);

}  // namespace pa
