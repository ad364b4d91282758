// Adam / AdamW update (runtime/backend.rs:1023-1075, kernels adam_moment :2545-2556 and
// adam_update :2558-2586) fused into one pass: read p, g, m, v and write p', m', v'
// (28 bytes per parameter instead of the reference's three kernels and three zero-fills).
// The expression order is the reference's, built with -ffp-contract=off, so the result is
// bit-identical to a sequential restatement of the three kernels.  The multi-tensor entry
// updates up to kMaxTensors tensors per launch, blocks split among them by size.
#include "common.hpp"

namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

// 512 lanes with one float4 of each stream per lane measured fastest for the 28 B/param stream
// (within 2% of a plain copy's rate on MI355X); more vectors per lane or smaller blocks lose 3-4%.
constexpr int kBlock = 512;
constexpr int kMaxTensors = 24;
constexpr int kVecPerThread = 1;  // float4 vectors per thread per block-chunk

struct AdamHyper {
    float lr, b1, b2, one_minus_b1, one_minus_b2, c1, c2, eps, wd;
};

__device__ __forceinline__ void adam_one(float &p, float g, float &m, float &v, float lr,
                                         const AdamHyper &h) {
    const float m_next = h.b1 * m + h.one_minus_b1 * g;
    const float gg = g * g;
    const float v_next = h.b2 * v + h.one_minus_b2 * gg;
    const float mh = m_next / h.c1;
    const float vh = v_next / h.c2;
    const float denom = sqrtf(vh) + h.eps;
    const float step = mh / denom + h.wd * p;
    p = p - lr * step;
    m = m_next;
    v = v_next;
}

struct AdamTensorArg {
    float *value;
    const float *gradient;
    float *first;
    float *second;
    const float *rates;
    int64_t len;
    int64_t block_begin;  // first block index of this tensor
    int32_t vec;          // 16-byte aligned and handled with float4
};

struct AdamMultiArgs {
    AdamTensorArg t[kMaxTensors];
    uint32_t first_block[kMaxTensors];  // t[i].block_begin, contiguous for one batch of scalar loads
    int32_t count;
    AdamHyper h;
};

__global__ void __launch_bounds__(kBlock) adam_multi_kernel(AdamMultiArgs args) {
    // Tensor of this block: a branch-free count over independent loads (no dependent chain).
    int ti = 0;
#pragma unroll
    for (int j = 1; j < kMaxTensors; ++j) ti += (j < args.count && blockIdx.x >= args.first_block[j]) ? 1 : 0;
    const AdamTensorArg &t = args.t[ti];
    const int64_t local_block = blockIdx.x - t.block_begin;
    constexpr int64_t per_block = (int64_t)kBlock * kVecPerThread * 4;  // elements per block
    const int64_t begin = local_block * per_block;
    const int64_t end = begin + per_block < t.len ? begin + per_block : t.len;
    const AdamHyper h = args.h;
    if (t.vec && !t.rates) {
        // Whole float4 vectors, lanes striding by the block so each access coalesces.  Every load
        // of the thread's kVecPerThread vectors is issued before any arithmetic, and the streams
        // bypass cache residency (each byte is touched once).
        const int64_t vbegin = begin / 4, vend = end / 4;
        floatx4 *__restrict__ pv = reinterpret_cast<floatx4 *>(t.value);
        const floatx4 *__restrict__ gv = reinterpret_cast<const floatx4 *>(t.gradient);
        floatx4 *__restrict__ mv = reinterpret_cast<floatx4 *>(t.first);
        floatx4 *__restrict__ vv = reinterpret_cast<floatx4 *>(t.second);
        floatx4 P[kVecPerThread], G[kVecPerThread], M[kVecPerThread], V[kVecPerThread];
#pragma unroll
        for (int u = 0; u < kVecPerThread; ++u) {
            const int64_t i = vbegin + threadIdx.x + (int64_t)u * kBlock;
            if (i < vend) {
                P[u] = __builtin_nontemporal_load(pv + i);
                G[u] = __builtin_nontemporal_load(gv + i);
                M[u] = __builtin_nontemporal_load(mv + i);
                V[u] = __builtin_nontemporal_load(vv + i);
            }
        }
#pragma unroll
        for (int u = 0; u < kVecPerThread; ++u) {
            const int64_t i = vbegin + threadIdx.x + (int64_t)u * kBlock;
            if (i < vend) {
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    float pc = P[u][c], mc = M[u][c], vc = V[u][c];
                    adam_one(pc, G[u][c], mc, vc, h.lr, h);
                    P[u][c] = pc;
                    M[u][c] = mc;
                    V[u][c] = vc;
                }
                __builtin_nontemporal_store(P[u], pv + i);
                __builtin_nontemporal_store(M[u], mv + i);
                __builtin_nontemporal_store(V[u], vv + i);
            }
        }
        for (int64_t i = vend * 4 + threadIdx.x; i < end; i += kBlock) {
            float p = t.value[i], m = t.first[i], v = t.second[i];
            adam_one(p, t.gradient[i], m, v, h.lr, h);
            t.value[i] = p;
            t.first[i] = m;
            t.second[i] = v;
        }
    } else {
        for (int64_t i = begin + threadIdx.x; i < end; i += kBlock) {
            float p = t.value[i], m = t.first[i], v = t.second[i];
            adam_one(p, t.gradient[i], m, v, t.rates ? t.rates[i] : h.lr, h);
            t.value[i] = p;
            t.first[i] = m;
            t.second[i] = v;
        }
    }
}

// Out-of-place single tensor (outputs may alias inputs).
__global__ void __launch_bounds__(kBlock) adam_kernel(const float *__restrict__ value,
                                                      const float *__restrict__ gradient,
                                                      const float *__restrict__ first,
                                                      const float *__restrict__ second,
                                                      const float *__restrict__ rates, int64_t len,
                                                      AdamHyper h, float *out_value, float *out_first,
                                                      float *out_second) {
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < len;
         i += (int64_t)gridDim.x * kBlock) {
        float p = value[i], m = first[i], v = second[i];
        adam_one(p, gradient[i], m, v, rates ? rates[i] : h.lr, h);
        out_value[i] = p;
        out_first[i] = m;
        out_second[i] = v;
    }
}

AdamHyper hyper(float lr, float b1, float b2, float c1, float c2, float eps, float wd) {
    AdamHyper h;
    h.lr = lr;
    h.b1 = b1;
    h.b2 = b2;
    h.one_minus_b1 = 1.0f - b1;
    h.one_minus_b2 = 1.0f - b2;
    h.c1 = c1;
    h.c2 = c2;
    h.eps = eps;
    h.wd = wd;
    return h;
}

// Muon's elementwise steps (model/optim.rs:644-669), each operation rounded as the reference's
// separate tensor ops round it (this file is built with -ffp-contract=off):
//   next = prev * momentum + g * (1 - momentum)          (prev absent: g * (1 - momentum))
//   direction = g * (1 - momentum) + next * momentum     (Nesterov; else next)
//   updated = p * decay - orthogonal * rate
template <bool PREV, bool NESTEROV>
__global__ void __launch_bounds__(256) muon_momentum_kernel(const float *__restrict__ g,
                                                            const float *__restrict__ prev, float *__restrict__ next,
                                                            float *__restrict__ direction, float momentum,
                                                            float observation, int64_t len) {
    for (int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4; i < len; i += (int64_t)gridDim.x * 1024) {
        if (i + 4 <= len) {
            const floatx4 gv = *reinterpret_cast<const floatx4 *>(g + i);
            floatx4 nv, dv;
            floatx4 pv = PREV ? *reinterpret_cast<const floatx4 *>(prev + i) : floatx4{};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float t2 = gv[e] * observation;
                nv[e] = PREV ? pv[e] * momentum + t2 : t2;
                dv[e] = NESTEROV ? t2 + nv[e] * momentum : nv[e];
            }
            *reinterpret_cast<floatx4 *>(next + i) = nv;
            if (NESTEROV) *reinterpret_cast<floatx4 *>(direction + i) = dv;
        } else {
            for (int64_t j = i; j < len; ++j) {
                const float t2 = g[j] * observation;
                const float n = PREV ? prev[j] * momentum + t2 : t2;
                next[j] = n;
                if (NESTEROV) direction[j] = t2 + n * momentum;
            }
        }
    }
}

__global__ void __launch_bounds__(256) muon_apply_kernel(const float *__restrict__ p,
                                                         const float *__restrict__ orthogonal,
                                                         float *__restrict__ out, float decay, float rate,
                                                         int64_t len) {
    for (int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4; i < len; i += (int64_t)gridDim.x * 1024) {
        if (i + 4 <= len) {
            const floatx4 pv = *reinterpret_cast<const floatx4 *>(p + i);
            const floatx4 ov = *reinterpret_cast<const floatx4 *>(orthogonal + i);
            floatx4 r;
#pragma unroll
            for (int e = 0; e < 4; ++e) r[e] = pv[e] * decay - ov[e] * rate;
            *reinterpret_cast<floatx4 *>(out + i) = r;
        } else {
            for (int64_t j = i; j < len; ++j) out[j] = p[j] * decay - orthogonal[j] * rate;
        }
    }
}

}  // namespace

extern "C" {

int axis_muon_momentum(axis_device device, const float *gradient, const float *previous, float *next,
                       float *direction, float momentum, int nesterov, int64_t len) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {gradient, 4 * len}, {previous, 4 * len}, {next, 4 * len}, {direction, 4 * len});
    AXIS_REQUIRE(len >= 0, "negative length");
    if (len == 0) return AXIS_OK;
    AXIS_REQUIRE(gradient && next && (direction || !nesterov), "null Muon buffer");
    AXIS_REQUIRE(axis::aligned16(gradient) && axis::aligned16(next) && (!previous || axis::aligned16(previous)) &&
                     (!nesterov || axis::aligned16(direction)),
                 "Muon buffers must be 16-byte aligned");
    const float observation = 1.0f - momentum;
    const unsigned blocks = axis::blocks_for((len + 3) / 4, 256, 8192);
    if (previous && nesterov)
        muon_momentum_kernel<true, true><<<blocks, 256, 0, device->stream>>>(gradient, previous, next, direction,
                                                                            momentum, observation, len);
    else if (previous)
        muon_momentum_kernel<true, false><<<blocks, 256, 0, device->stream>>>(gradient, previous, next, direction,
                                                                             momentum, observation, len);
    else if (nesterov)
        muon_momentum_kernel<false, true><<<blocks, 256, 0, device->stream>>>(gradient, previous, next, direction,
                                                                             momentum, observation, len);
    else
        muon_momentum_kernel<false, false><<<blocks, 256, 0, device->stream>>>(gradient, previous, next,
                                                                              direction, momentum, observation, len);
    return axis::launch_status("muon_momentum_kernel");
}

int axis_muon_apply(axis_device device, const float *value, const float *orthogonal, float *out, float decay,
                    float rate, int64_t len) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {value, 4 * len}, {orthogonal, 4 * len}, {out, 4 * len});
    AXIS_REQUIRE(len >= 0, "negative length");
    if (len == 0) return AXIS_OK;
    AXIS_REQUIRE(value && orthogonal && out, "null Muon buffer");
    AXIS_REQUIRE(axis::aligned16(value) && axis::aligned16(orthogonal) && axis::aligned16(out),
                 "Muon buffers must be 16-byte aligned");
    muon_apply_kernel<<<axis::blocks_for((len + 3) / 4, 256, 8192), 256, 0, device->stream>>>(value, orthogonal, out,
                                                                                             decay, rate, len);
    return axis::launch_status("muon_apply_kernel");
}

int axis_adam(axis_device device, const float *value, const float *gradient, const float *first,
              const float *second, const float *learning_rates, int64_t len, float learning_rate,
              float beta1, float beta2, float correction1, float correction2, float epsilon,
              float weight_decay, float *out_value, float *out_first, float *out_second) {
    AXIS_ENTER(device);
    AXIS_GUARD(device, {value, 4 * len}, {gradient, 4 * len}, {first, 4 * len}, {second, 4 * len}, {learning_rates, 4 * len}, {out_value, 4 * len}, {out_first, 4 * len}, {out_second, 4 * len});
    AXIS_REQUIRE(len >= 0, "negative length");
    if (len == 0) return AXIS_OK;
    AXIS_REQUIRE(value && gradient && first && second && out_value && out_first && out_second,
                 "null adam buffer");
    const AdamHyper h = hyper(learning_rate, beta1, beta2, correction1, correction2, epsilon,
                              weight_decay);
    adam_kernel<<<axis::blocks_for(len, kBlock, (int64_t)device->multiprocessors * 16), kBlock, 0,
                  device->stream>>>(value, gradient, first, second, learning_rates, len, h,
                                    out_value, out_first, out_second);
    return axis::launch_status("adam_kernel");
}

int axis_adam_multi(axis_device device, const axis_adam_tensor *tensors, int32_t count,
                    float learning_rate, float beta1, float beta2, float correction1,
                    float correction2, float epsilon, float weight_decay) {
    AXIS_ENTER(device);
    AXIS_REQUIRE(count >= 0 && (count == 0 || tensors), "bad adam_multi tensor list");
    for (int32_t i = 0; i < count; ++i) {
        const axis_adam_tensor &t = tensors[i];
        AXIS_REQUIRE(t.len >= 0, "negative adam tensor length");
        AXIS_REQUIRE(t.len == 0 || (t.value && t.gradient && t.first && t.second),
                     "null adam tensor buffer");
        AXIS_GUARD(device, {t.value, 4 * t.len}, {t.gradient, 4 * t.len}, {t.first, 4 * t.len},
                   {t.second, 4 * t.len}, {t.learning_rates, 4 * t.len});
    }
    const AdamHyper h = hyper(learning_rate, beta1, beta2, correction1, correction2, epsilon,
                              weight_decay);
    constexpr int64_t per_block = (int64_t)kBlock * kVecPerThread * 4;
    int32_t i = 0;
    while (i < count) {
        AdamMultiArgs args{};
        args.h = h;
        int64_t blocks = 0;
        int32_t n = 0;
        for (; i < count && n < kMaxTensors; ++i) {
            const axis_adam_tensor &t = tensors[i];
            if (t.len == 0) continue;
            AdamTensorArg &a = args.t[n++];
            a.value = t.value;
            a.gradient = t.gradient;
            a.first = t.first;
            a.second = t.second;
            a.rates = t.learning_rates;
            a.len = t.len;
            a.block_begin = blocks;
            args.first_block[n - 1] = (uint32_t)blocks;
            a.vec = axis::aligned16(t.value) && axis::aligned16(t.gradient) &&
                    axis::aligned16(t.first) && axis::aligned16(t.second);
            blocks += (t.len + per_block - 1) / per_block;
        }
        if (n == 0) continue;
        AXIS_REQUIRE(blocks < INT32_MAX, "adam_multi launch too large");
        args.count = n;
        double bytes = 0.0;  // algorithmic: read p, g, m, v (+ rate), write p, m, v
        for (int32_t t = 0; t < n; ++t) bytes += (args.t[t].rates ? 32.0 : 28.0) * (double)args.t[t].len;
        axis::TimedLaunch timed(device, "adam", bytes);
        adam_multi_kernel<<<(unsigned)blocks, kBlock, 0, device->stream>>>(args);
        if (int s = axis::launch_status("adam_multi_kernel")) return s;
    }
    return AXIS_OK;
}

}  // extern "C"
