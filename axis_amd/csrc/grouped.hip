// CSR plan reductions (runtime/backend.rs:1089-1125, :1365-1440; kernels :2964-3116).
//
// grouped: stage one sums each chunk of <= 512 contributions sequentially (one lane per chunk),
// stage two sums a group's chunk partials in chunk order and scales once -- the reference's
// exact association, so results are bit-identical to a sequential restatement.
// grouped_minimum/maximum: one lane per group walks its members in plan order keeping the first
// strictly better finite value; the winner mask is one lane per input position.
#include <cfloat>

#include "common.hpp"

namespace {

template <bool PRODUCT>
__global__ void __launch_bounds__(256) grouped_partial_kernel(
    const float *__restrict__ a, const float *__restrict__ b, const int32_t *__restrict__ chunk_offsets,
    const int32_t *__restrict__ left, const int32_t *__restrict__ right, float *__restrict__ partial,
    int64_t chunks) {
    const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (c >= chunks) return;
    const int32_t start = chunk_offsets[c], end = chunk_offsets[c + 1];
    float sum = 0.0f;
    for (int32_t i = start; i < end; ++i) {
        const float value = a[left[i]];
        if (PRODUCT) {
            const float product = value * b[right[i]];
            sum = sum + product;
        } else {
            sum = sum + value;
        }
    }
    partial[c] = sum;
}

__global__ void __launch_bounds__(256) grouped_combine_kernel(const float *__restrict__ partial,
                                                              const int32_t *__restrict__ chunk_group,
                                                              float scale, float *__restrict__ out,
                                                              int64_t groups) {
    const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (g >= groups) return;
    float sum = 0.0f;
    for (int32_t c = chunk_group[g]; c < chunk_group[g + 1]; ++c) sum = sum + partial[c];
    out[g] = sum * scale;
}

template <bool MAXIMUM>
__global__ void __launch_bounds__(256) grouped_extreme_kernel(const float *__restrict__ a,
                                                              const int32_t *__restrict__ offsets,
                                                              const int32_t *__restrict__ left,
                                                              float *__restrict__ out,
                                                              int32_t *__restrict__ winners,
                                                              int64_t groups) {
    const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (g >= groups) return;
    int32_t winner = -1;
    float best = MAXIMUM ? -INFINITY : INFINITY;
    for (int32_t i = offsets[g]; i < offsets[g + 1]; ++i) {
        const int32_t candidate = left[i];
        const float value = a[candidate];
        const bool finite = value >= -FLT_MAX && value <= FLT_MAX;
        const bool better = MAXIMUM ? value > best : value < best;
        if (finite && better) {
            best = value;
            winner = candidate;
        }
    }
    winners[g] = winner;
    const bool found = MAXIMUM ? best >= -FLT_MAX : best <= FLT_MAX;
    out[g] = found ? best : __builtin_nanf("");
}

__global__ void __launch_bounds__(256) winner_mask_kernel(const int32_t *__restrict__ winners,
                                                          const int32_t *__restrict__ group_of,
                                                          float *__restrict__ mask, int64_t len) {
    const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (p >= len) return;
    mask[p] = winners[group_of[p]] == p ? 1.0f : 0.0f;
}

template <bool MAXIMUM>
int grouped_extreme(axis_device device, const float *a, int64_t input_len, axis_plan forward,
                    axis_plan reverse, float *out, int32_t *winners, float *winner_mask) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {a, 4 * input_len}, {out, 1}, {winners, 1}, {winner_mask, 1});
    AXIS_REQUIRE(a && forward && reverse && out && winner_mask, "null grouped extreme argument");
    AXIS_REQUIRE(reverse->count == input_len && reverse->groups == input_len,
                 "reverse plan must be a gather plan over every input position");
    axis::Scratch scratch;
    int32_t *w = winners;
    if (!w) {
        if (int s = scratch.get(device, sizeof(int32_t) * (size_t)forward->groups)) return s;
        w = scratch.as<int32_t>();
    }
    grouped_extreme_kernel<MAXIMUM><<<axis::blocks_for(forward->groups, 256, INT32_MAX), 256, 0,
                                      device->stream>>>(a, forward->offsets, forward->left, out, w,
                                                        forward->groups);
    if (int s = axis::launch_status("grouped_extreme_kernel")) return s;
    winner_mask_kernel<<<axis::blocks_for(input_len, 256, INT32_MAX), 256, 0, device->stream>>>(
        w, reverse->left, winner_mask, input_len);
    return axis::launch_status("winner_mask_kernel");
}

}  // namespace

extern "C" {

int axis_grouped(axis_device device, const float *a, const float *b, axis_plan plan, float scale,
                 float *out) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {a, 1}, {b, 1}, {out, 1});
    AXIS_REQUIRE(a && plan && out, "null grouped argument");
    AXIS_REQUIRE(!b || plan->right, "a product reduction needs a plan with right indices");
    axis::Scratch partial;
    if (plan->chunks > 0) {
        if (int s = partial.get(device, sizeof(float) * (size_t)plan->chunks)) return s;
        if (b)
            grouped_partial_kernel<true><<<axis::blocks_for(plan->chunks, 256, INT32_MAX), 256, 0,
                                           device->stream>>>(a, b, plan->chunk_offsets, plan->left,
                                                             plan->right, partial.as<float>(),
                                                             plan->chunks);
        else
            grouped_partial_kernel<false><<<axis::blocks_for(plan->chunks, 256, INT32_MAX), 256, 0,
                                            device->stream>>>(a, a, plan->chunk_offsets, plan->left,
                                                              plan->left, partial.as<float>(),
                                                              plan->chunks);
        if (int s = axis::launch_status("grouped_partial_kernel")) return s;
    }
    grouped_combine_kernel<<<axis::blocks_for(plan->groups, 256, INT32_MAX), 256, 0, device->stream>>>(
        partial.as<float>(), plan->chunk_group, scale, out, plan->groups);
    return axis::launch_status("grouped_combine_kernel");
}

int axis_grouped_minimum(axis_device device, const float *a, int64_t input_len, axis_plan forward,
                         axis_plan reverse, float *out, int32_t *winners, float *winner_mask) {
    return grouped_extreme<false>(device, a, input_len, forward, reverse, out, winners, winner_mask);
}

int axis_grouped_maximum(axis_device device, const float *a, int64_t input_len, axis_plan forward,
                         axis_plan reverse, float *out, int32_t *winners, float *winner_mask) {
    return grouped_extreme<true>(device, a, input_len, forward, reverse, out, winners, winner_mask);
}

}  // extern "C"
