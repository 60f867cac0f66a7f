/* nda_device.h - device helpers shared by the gfx950 kernels. */
#pragma once

#include "nda_internal.h"

namespace nda {

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float sigmoid_dev(float x) { return 1.0f / (1.0f + __expf(-x)); }

// Which positions a row sees (the dispatch arithmetic of attention(),
// engine/src/nd_model.c:2451-2483), split into the shared-prefix run and
// the sequence's own slots. Own slots [0, n_own) are contiguous: without a
// shared prefix they are the sinks [0, n_sink) followed by the ring
// [n_sink, n_sink + rcount); with one they are ring indices [0, rcount).
struct Visible {
    int n_sh, n_own;
};

__device__ __forceinline__ Visible visible(const SeqDev &s, int p, int window)
{
    int sinks = min(s.n_sink, p + 1);
    int rcap = window - s.n_sink;
    int rcount = (p + 1 <= s.n_sink) ? 0 : min(p + 1 - s.n_sink, rcap);
    Visible v;
    v.n_sh = s.prefix >= 0 ? sinks : 0;
    v.n_own = s.prefix >= 0 ? rcount : sinks + rcount;
    return v;
}

// Own slot of position p (kv_slot, engine/src/nd_model.c:1302-1309, with the
// sinks of a shared prefix living outside the sequence's pages).
__device__ __forceinline__ int own_slot(const SeqDev &s, int p, int window)
{
    if (s.prefix >= 0)
        return (p - s.n_sink) % (window - s.n_sink);
    if (p < s.n_sink)
        return p;
    return s.n_sink + (p - s.n_sink) % (window - s.n_sink);
}

} // namespace nda
