// The general attention kernels (attention_any.hip): float32/float16/bfloat16,
// head dims up to 512, any strides, and the score gradient for the bias
// gradient. tvk_attention_fwd / tvk_attention_bwd run them for every case the
// MFMA kernels of attention.hip do not take.
#pragma once

#include "tvk_common.h"

namespace tvk {

struct AnyAttnArgs {
    const void* q;
    const void* k;
    const void* v;
    const void* bias;
    void* out;
    float* lse;
    const void* dout;
    void* dq;
    void* dk;
    void* dv;
    float* ds;      // score gradient [B, Hq, L, S] (float32), or NULL
    float* delta;   // rowsum(dout * out), [B][Hq][L]
    int64_t sq[4], sk[4], sv[4], sb[4], so[4], sl[3];
    int64_t sdo[4], sdq[4], sdk[4], sdv[4], sds[4];
    int B, Hq, group, L, S, D, Dv;
    int causal;
    float scale;
    int64_t es;     // element size of q, k, v, bias, out, dout and the gradients
};

// True when the general kernels take the case's dtype and sizes.
bool attn_any_applies(const tvk_attention_desc* d);
tvk_status attn_any_fwd(const tvk_attention_desc* d, hipStream_t s);
// `delta` holds batch * heads_q * len_q floats of scratch for the call.
tvk_status attn_any_bwd(const tvk_attention_bwd_desc* desc, float* delta, hipStream_t s);

}  // namespace tvk
