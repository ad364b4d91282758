// The reference's max-pool winner over one 2x2 window of ReLU outputs (Tensor::min over the
// negated window, runtime/backend.rs:3019-3056, tensor.rs:2880-2946): the first strictly greater
// finite value in window order (ky major, kx minor); NaN and winner 255 when no value is finite.
#pragma once

#include <hip/hip_runtime.h>

#include <cfloat>

// y[e] = pre-activation at window position e; best = pooled ReLU value, winner = its position.
// ReLU maps NaN and every non-positive value to +0, so the candidates are +0, positive finite
// values and +inf; without +inf the winner is the first position equal to the maximum.
__device__ __forceinline__ void relu_pool_window4(const float y[4], float &best, int &winner) {
    float r[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = y[e] > 0.0f ? y[e] : 0.0f;
    best = __builtin_fmaxf(__builtin_fmaxf(__builtin_fmaxf(r[0], r[1]), r[2]), r[3]);
    winner = r[2] == best ? 2 : 3;
    winner = r[1] == best ? 1 : winner;
    winner = r[0] == best ? 0 : winner;
    if (best > FLT_MAX) {  // an infinite candidate: the exact scan
        best = -INFINITY;
        winner = 255;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (r[e] <= FLT_MAX && r[e] > best) {
                best = r[e];
                winner = e;
            }
        if (winner == 255) best = __builtin_nanf("");
    }
}
