// The reference's max-pool winner over one 2x2 window of ReLU outputs (Tensor::min over the
// negated window, runtime/backend.rs:3019-3056, tensor.rs:2880-2946): the first strictly greater
// finite value in window order (ky major, kx minor); NaN and winner 255 when no value is finite.
#pragma once

#include <hip/hip_runtime.h>

#include <cfloat>

// y[e] = pre-activation at window position e; best = pooled ReLU value, winner = its position.
// ReLU maps NaN and every non-positive value to +0, so the candidates are +0, positive finite
// values and +inf.  With m the largest non-NaN y: when m > 0 is finite the winner is the first
// position holding m (only a positive y equals m); otherwise every candidate is +0 and position 0
// wins with +0; an infinite m takes the exact scan.
__device__ __forceinline__ void relu_pool_window4(const float y[4], float &best, int &winner) {
    const float m = __builtin_fmaxf(__builtin_fmaxf(__builtin_fmaxf(y[0], y[1]), y[2]), y[3]);
    const bool positive = m > 0.0f;
    best = positive ? m : 0.0f;
    int w = y[2] == m ? 2 : 3;
    w = y[1] == m ? 1 : w;
    w = y[0] == m ? 0 : w;
    winner = positive ? w : 0;
    if (m > FLT_MAX) {  // an infinite candidate: the exact scan over the ReLU values
        best = -INFINITY;
        winner = 255;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float r = y[e] > 0.0f ? y[e] : 0.0f;
            if (r <= FLT_MAX && r > best) {
                best = r;
                winner = e;
            }
        }
        if (winner == 255) best = __builtin_nanf("");
    }
}
