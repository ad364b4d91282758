// Adam / AdamW (model/optim.rs:9-226), Muon and MuonWithAuxAdamW (optim.rs:440-800), and the
// Trainer step (runtime/train.rs:231-275).
//
// Adam keeps the reference's out-of-place contract (prepare builds every new value, commit swaps
// them in), but when a parameter's value and moments are owned by nothing else -- so no live
// Tensor could observe the change -- all such tensors are updated in place by one multi-tensor
// launch (28 bytes per parameter).  Validation happens before any launch, so an error leaves
// parameters, moments and the step counter untouched.
#include <algorithm>
#include <cmath>
#include <set>
#include <unordered_set>

#include "axis.hpp"

namespace axis {

namespace {

void validate_adam(float lr, float b1, float b2, float eps) {
    if (!std::isfinite(lr) || lr <= 0.0f) raise("Adam learning rate must be finite and positive");
    if (!std::isfinite(b1) || b1 < 0.0f || b1 >= 1.0f) raise("Adam beta1 must be finite and within 0..1");
    if (!std::isfinite(b2) || b2 < 0.0f || b2 >= 1.0f) raise("Adam beta2 must be finite and within 0..1");
    if (!std::isfinite(eps) || eps <= 0.0f) raise("Adam epsilon must be finite and positive");
}

}  // namespace

// ------------------------------------------------------------------ Adam

Adam::Adam(float lr, float b1, float b2, float eps)
    : learning_rate(lr), beta1(b1), beta2(b2), epsilon(eps) {
    validate_adam(lr, b1, b2, eps);
}

AdamW::AdamW(float lr, float wd, float b1, float b2, float eps) : Adam(lr, b1, b2, eps) {
    if (!std::isfinite(wd) || wd < 0.0f) raise("AdamW weight decay must be finite and nonnegative");
    weight_decay = wd;
}

void Adam::set_learning_rate(float lr) {
    if (!std::isfinite(lr) || lr <= 0.0f) raise("Adam learning rate must be finite and positive");
    learning_rate = lr;
}

Adam::Prepared Adam::prepare(const std::vector<Parameter> &parameters) const {
    double started = now_seconds();
    if (step_count == std::numeric_limits<int32_t>::max()) raise("Adam step overflow");
    Prepared prepared;
    prepared.next_step = step_count + 1;
    const float c1 = 1.0f - powi(beta1, prepared.next_step);
    const float c2 = 1.0f - powi(beta2, prepared.next_step);
    std::vector<Parameter> unique;
    std::unordered_set<uint64_t> seen;
    for (auto &p : parameters) {
        if (!seen.insert(p.id()).second) continue;
        if (!p.s->tensor.n->grad) raise("parameter has no gradient; run backward before step");
        unique.push_back(p);
    }
    if (unique.empty()) return prepared;
    const Device dev = unique.front().tensor().device();
    std::vector<axis_adam_tensor> in_place;
    for (auto &p : unique) {
        const Tensor t = p.tensor();
        const Buffer &g = t.n->grad;
        auto found = states.find(p.id());
        State st;
        bool fresh = found == states.end();
        if (fresh) {
            st.first = dev.zeros_buffer(t.shape().len);
            st.second = dev.zeros_buffer(t.shape().len);
        } else {
            st = found->second;
        }
        // In place only when nothing but the parameter (and this call) can reach the value and
        // nothing but this optimizer holds the moments.
        bool own_value = p.s->tensor.n.use_count() <= 2 && t.value().use_count() == 1;
        bool own_moments = fresh || (found->second.first.use_count() <= 2 &&
                                     found->second.second.use_count() <= 2);
        Update u;
        u.parameter = p;
        if (own_value && own_moments) {
            in_place.push_back(axis_adam_tensor{t.value()->f32(), g->f32(), st.first->f32(),
                                                st.second->f32(), nullptr, t.shape().len});
            u.tensor = Tensor::node(t.shape(), t.layout(), t.value(), dev, {}, false);
            u.state = st;
        } else {
            Buffer value = dev.alloc(t.shape().len), m = dev.alloc(t.shape().len),
                   v = dev.alloc(t.shape().len);
            check(axis_adam(dev.h(), t.value()->f32(), g->f32(), st.first->f32(), st.second->f32(),
                            nullptr, t.shape().len, learning_rate, beta1, beta2, c1, c2, epsilon,
                            weight_decay, value->f32(), m->f32(), v->f32()),
                  "adam");
            u.tensor = Tensor::node(t.shape(), t.layout(), value, dev, {}, false);
            u.state = State{m, v};
        }
        prepared.updates.push_back(std::move(u));
    }
    if (!in_place.empty())
        check(axis_adam_multi(dev.h(), in_place.data(), (int32_t)in_place.size(), learning_rate,
                              beta1, beta2, c1, c2, epsilon, weight_decay),
              "adam_multi");
    profile("adam_prepare", started);
    return prepared;
}

void Adam::commit(Prepared &&prepared) {
    for (auto &u : prepared.updates) {
        u.parameter.replace(u.tensor);
        states[u.parameter.id()] = u.state;
    }
    step_count = prepared.next_step;
}

void Adam::step_parameters(const std::vector<Parameter> &parameters) { commit(prepare(parameters)); }

// ------------------------------------------------------------------ Muon

namespace {
constexpr float kNsA = 3.4445f, kNsB = -4.7750f, kNsC = 2.0315f;
constexpr int kNsSteps = 5;
constexpr float kNormalizationEpsilon = 1e-7f;
}  // namespace

Muon::Muon(const std::vector<MuonMatrix> &sel, float lr, float mu, bool nest, float wd)
    : learning_rate(lr), momentum(mu), nesterov(nest), weight_decay(wd) {
    if (!std::isfinite(lr) || lr <= 0.0f) raise("Muon learning rate must be finite and positive");
    if (!std::isfinite(mu) || mu < 0.0f || mu >= 1.0f) raise("Muon momentum must be finite and within 0..1");
    if (!std::isfinite(wd) || wd < 0.0f) raise("Muon weight decay must be finite and nonnegative");
    for (auto &m : sel) {
        auto it = selected.find(m.id);
        if (it != selected.end() && it->second != m.orientation)
            raise("Muon parameter " + std::to_string(m.id) +
                  " was selected with conflicting matrix orientations");
        selected[m.id] = m.orientation;
    }
    if (selected.empty()) raise("Muon requires at least one explicit matrix selection");
}

std::pair<std::vector<Muon::Selected>, std::vector<Parameter>> Muon::partition(Module &model) const {
    std::unordered_set<uint64_t> seen, found;
    std::vector<Selected> muon;
    std::vector<Parameter> aux;
    for (auto &p : model.parameters()) {
        if (!seen.insert(p.id()).second) continue;
        auto it = selected.find(p.id());
        if (it != selected.end()) {
            found.insert(p.id());
            muon.push_back(Selected{p, it->second});
        } else {
            aux.push_back(p);
        }
    }
    if (found.size() != selected.size())
        raise("Muon selection contains " + std::to_string(selected.size() - found.size()) +
              " ParamId(s) that do not belong to this model");
    return {muon, aux};
}

void Muon::step(Module &model) {
    auto [params, aux] = partition(model);
    if (!aux.empty())
        raise("Muon selection omits " + std::to_string(aux.size()) +
              " unique model parameter(s); use MuonWithAuxAdamW for an auxiliary remainder");
    commit(prepare(params));
}

Muon::Prepared Muon::prepare(const std::vector<Selected> &parameters) const {
    double started = now_seconds();
    Prepared prepared;
    prepared.next_step = step_count + 1;
    for (auto &s : parameters) {
        if (s.parameter.tensor().shape().rank() != 2)
            raise("Muon parameter " + std::to_string(s.parameter.id()) + " must have rank 2; observed rank " +
                  std::to_string(s.parameter.tensor().shape().rank()));
        if (!s.parameter.grad())
            raise("Muon parameter " + std::to_string(s.parameter.id()) +
                  " has no gradient; run backward before step");
    }
    if (parameters.empty()) raise("Muon requires at least one selected rank-2 parameter");
    // One contiguous layout shared by every operand: the elementwise steps run as one pass each
    // (axis_muon_momentum / axis_muon_apply, the same roundings as the op sequence below).
    auto plain = [](const Tensor &t, const Tensor &like) {
        return t.shape() == like.shape() && t.layout() == Layout::contiguous(t.shape()) && t.value() &&
               t.value()->floats() == t.shape().len && !t.requires_grad();
    };
    for (auto &s : parameters) {
        Tensor gradient = *s.parameter.grad();
        const float observation_weight = 1.0f - momentum;
        auto prev = states.find(s.parameter.id());
        Tensor next_momentum, direction;
        if (plain(gradient, gradient) && (prev == states.end() || plain(prev->second, gradient))) {
            const Device &dev = gradient.device();
            const int64_t len = gradient.shape().len;
            Buffer next = dev.alloc(len);
            Buffer dir = nesterov ? dev.alloc(len) : Buffer();
            check(axis_muon_momentum(dev.h(), gradient.value()->f32(),
                                     prev != states.end() ? prev->second.value()->f32() : nullptr, next->f32(),
                                     dir ? dir->f32() : nullptr, momentum, nesterov ? 1 : 0, len),
                  "muon_momentum");
            next_momentum = Tensor::node(gradient.shape(), gradient.layout(), next, dev, {}, false);
            direction = nesterov ? Tensor::node(gradient.shape(), gradient.layout(), dir, dev, {}, false)
                                 : next_momentum;
        } else {
            next_momentum = prev != states.end()
                                ? prev->second.scale(momentum).add(gradient.scale(observation_weight))
                                : gradient.scale(observation_weight);
            direction = nesterov ? gradient.scale(observation_weight).add(next_momentum.scale(momentum))
                                 : next_momentum;
        }
        Tensor orthogonal = zeroth_power(direction);
        Tensor p = s.parameter.tensor();
        const auto &dims = p.shape().dims;
        int64_t fan_in = s.orientation == MuonOrientation::FanInFanOut ? dims[0].extent : dims[1].extent;
        int64_t fan_out = s.orientation == MuonOrientation::FanInFanOut ? dims[1].extent : dims[0].extent;
        const float scaling = std::sqrt(std::max((float)fan_out / (float)fan_in, 1.0f));
        const float decay = 1.0f - learning_rate * weight_decay;
        const float rate = learning_rate * scaling;
        Tensor updated;
        Tensor held = p.detach();
        if (plain(held, held) && plain(orthogonal, held)) {
            const Device &dev = held.device();
            Buffer out = dev.alloc(held.shape().len);
            check(axis_muon_apply(dev.h(), held.value()->f32(), orthogonal.value()->f32(), out->f32(), decay, rate,
                                  held.shape().len),
                  "muon_apply");
            updated = Tensor::node(held.shape(), held.layout(), out, dev, {}, false);
        } else {
            updated = held.scale(decay).sub(orthogonal.scale(rate));
        }
        prepared.updates.push_back(Update{s.parameter, updated, next_momentum});
    }
    profile("muon_prepare", started);
    return prepared;
}

void Muon::commit(Prepared &&prepared) {
    for (auto &u : prepared.updates) {
        u.parameter.replace(u.tensor);
        states[u.parameter.id()] = u.momentum;
    }
    step_count = prepared.next_step;
}

// optim.rs:728-752
Tensor zeroth_power(const Tensor &matrix) {
    const auto &dims = matrix.shape().dims;
    Axis row = dims[0].axis, column = dims[1].axis;
    Axis small = dims[0].extent <= dims[1].extent ? row : column;
    Axis large = dims[0].extent <= dims[1].extent ? column : row;
    Axis inner = small.role("muon_ns_inner");
    Axis output = small.role("muon_ns_output");
    Tensor x = matrix.normalized_l2(kNormalizationEpsilon);
    if (!x.requires_grad()) {
        // No gradient flows through the orthogonalisation, so the iteration runs on x held
        // [small, large] row-major: gram = x.x^T through the NT kernel (no transpose copy), and each
        // scale-and-add folds into its product's epilogue with the same roundings:
        //   b  = kNsB * gram + kNsC * (gram . gram)      (gram_squared of the lowering below)
        //   x' = kNsA * x + b . x
        if (!(x.layout() == Layout::make(x.shape(), {small, large}))) x = x.with_layout({small, large});
        const Device dev = x.device();  // a copy: x is reassigned below
        const int64_t s = x.extent(small), l = x.extent(large);
        for (int i = 0; i < kNsSteps; ++i) {
            Tensor gram = x.contract(x.rename(small, inner), {large});
            Buffer b = dev.matmul_axpby(gram.value(), gram.value(), gram.value(), 1, s, s, s, kNsC, kNsB);
            Buffer next = dev.matmul_axpby(b, x.value(), x.value(), 1, s, s, l, 1.0f, kNsA);
            x = Tensor::node(x.shape(), x.layout(), next, dev, {}, false);
        }
        return x;
    }
    for (int i = 0; i < kNsSteps; ++i) {
        Tensor gram = x.contract(x.rename(small, inner), {large});
        Tensor gram_rhs = gram.rename(inner, output).rename(small, inner);
        Tensor gram_squared = gram.contract(gram_rhs, {inner}).rename(output, inner);
        Tensor b = gram.scale(kNsB).add(gram_squared.scale(kNsC));
        Tensor bx = b.contract(x.rename(small, inner), {inner});
        x = x.scale(kNsA).add(bx);
    }
    return x;
}

MuonWithAuxAdamW::MuonWithAuxAdamW(const std::vector<MuonMatrix> &sel, float muon_lr, float adamw_lr,
                                   float wd)
    : muon(sel, muon_lr, 0.95f, true, wd), adamw(adamw_lr, wd) {}

void MuonWithAuxAdamW::step(Module &model) {
    auto [muon_params, aux] = muon.partition(model);
    // Prepare both arms before either optimizer mutates parameters or state.
    auto m = muon.prepare(muon_params);
    auto a = adamw.prepare(aux);
    muon.commit(std::move(m));
    adamw.commit(std::move(a));
}

// ------------------------------------------------------------------ Trainer (train.rs:231-275)

TrainStep Trainer::step(Module &model, const std::function<Tensor(Module &)> &loss_fn) {
    double started = now_seconds();
    model.zero_grad();
    profile("train_zero_grad", started);
    started = now_seconds();
    Tensor loss = loss_fn(model);
    profile("train_loss", started);
    if (loss.shape().rank() != 0)
        raise("Trainer loss closure must return a scalar; reduce loss axes explicitly");
    started = now_seconds();
    loss.backward();
    profile("train_backward", started);
    started = now_seconds();
    optimizer->step(model);
    profile("train_optimizer", started);
    started = now_seconds();
    loss.device().synchronize();
    profile("train_boundary", started);
    completed += 1;
    return TrainStep{completed, loss};
}

}  // namespace axis
