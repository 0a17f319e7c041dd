// attn_generic.hpp — the attention path for head sizes and query groupings
// the tuned decode and prefill kernels do not take (attn_generic.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "ikv_common.hpp"

namespace ikv {

constexpr int kGenericMaxDim = 512;  // largest head_dim of the generic path

// Whether attn_generic takes the shape: n_head a multiple of n_head_kv, and
// 1 <= head_dim <= kGenericMaxDim.
bool generic_attn_shape(int n_head, int n_head_kv, int head_dim);

// out[t][h] = causal GQA attention of query rows q[t][h] (t < n_q) over keys
// [0, min(n_kv, n_past + t + 1)) of k / v ([n_kv][n_head_kv][head_dim], or a
// paged pool read through `pages`); scale <= 0 means 1/sqrt(head_dim).
// Any alignment; no workspace. 0, -ENOTSUP / -EINVAL / -EOVERFLOW before the
// launch, or the launch's hipError_t.
int attn_generic(const float *q, const float *k, const float *v, const Pages *pages, float *out,
                 int n_head, int n_head_kv, int head_dim, int64_t n_q, int64_t n_kv,
                 int64_t n_past, float scale, hipStream_t s);

// One query token (a decode step) over keys [0, n_kv): the same result as
// attn_generic with n_q = 1 and n_past = n_kv - 1 (within the path's float
// tolerance, not bitwise: the context is split over workgroups, each serving
// every query head of its KV head, and the splits are merged in order by a
// second launch). The split form needs workspace_bytes >=
// generic_decode_ws_bytes(...) of 16-byte aligned device memory and
// n_head / n_head_kv * ceil(head_dim / 64) <= 32 (rounded to 1, 2, 4, 8
// dims per lane); otherwise (or with no workspace) attn_generic runs.
size_t generic_decode_ws_bytes(int n_head, int n_head_kv, int head_dim, int64_t n_kv);
int attn_generic_decode(const float *q, const float *k, const float *v, const Pages *pages,
                        float *out, int n_head, int n_head_kv, int head_dim, int64_t n_kv,
                        float scale, void *workspace, size_t workspace_bytes, hipStream_t s);

}  // namespace ikv
