// DPM-Solver++ of the drop-in API.  The arithmetic is the one the reference
// performs (src/scheduler.cpp:89-318), kept in the same fp32 operation order
// so a denoise loop driven by this scheduler follows the reference's latents:
//   sigma_i   = shift * s / (1 + (shift - 1) * s),  s = 1 - (1 + (1/T - 1) * i/n)
//   timestep  = int(sigma * T)                      (flipped, sigma_n = 0 appended)
//   x0        = sample - sigma_t * v                (flow prediction)
//   lambda    = log(1 - sigma) - log(sigma)
//   1st order : (sigma_t/sigma_s) x + (-(1 - sigma_t)(e^-h - 1)) x0
//   2nd order : (sigma_t/sigma_s0) x + (-(1 - sigma_t)(e^-h - 1)) m0
//               + (-0.5 (1 - sigma_t)(e^-h - 1)) (m0 - m1) / r0,  r0 = h0 / h
#include "scheduler.h"

#include <cmath>
#include <stdexcept>

namespace {

void check_config(const SanaSchedulerConfig & c) {
    if (c.solver_order == 0) throw std::invalid_argument("solver_order must be positive");
    if (c.solver_order > 2) throw std::invalid_argument("only solver_order <= 2 is supported");
    if (c.prediction_type != "flow_prediction") throw std::invalid_argument("only flow_prediction is supported");
    if (c.algorithm_type != "dpmsolver++") throw std::invalid_argument("only dpmsolver++ is supported");
    if (c.solver_type != "midpoint" && c.solver_type != "heun")
        throw std::invalid_argument("solver_type must be midpoint or heun");
}

void check_step(const SanaSchedulerState & st) {
    if (st.schedule.timesteps.empty()) throw std::invalid_argument("scheduler state has no timesteps");
    if (st.schedule.sigmas.size() != st.schedule.timesteps.size() + 1)
        throw std::invalid_argument("scheduler sigmas must have one extra final entry");
    if (st.step_index >= st.schedule.timesteps.size())
        throw std::invalid_argument("scheduler step_index is out of range");
}

// (alpha_t, sigma_t) of a flow sigma, or of a VP sigma when flow sigmas are off.
void alpha_sigma(float sigma, const SanaSchedulerConfig & c, float & alpha, float & sig) {
    if (c.use_flow_sigmas) {
        alpha = 1.0f - sigma;
        sig = sigma;
    } else {
        alpha = 1.0f / std::sqrt(sigma * sigma + 1.0f);
        sig = sigma * alpha;
    }
}

float lambda_of(float alpha, float sigma) { return std::log(alpha) - std::log(sigma); }

}  // namespace

SanaSchedulerConfig make_sana_scheduler_config() { return SanaSchedulerConfig(); }

SanaSchedulerTimesteps build_sana_scheduler_timesteps(size_t n, const SanaSchedulerConfig & c) {
    check_config(c);
    if (n == 0) throw std::invalid_argument("num_inference_steps must be positive");
    if (!c.use_flow_sigmas) throw std::invalid_argument("only use_flow_sigmas=true is supported");
    if (c.timestep_spacing != "linspace") throw std::invalid_argument("only linspace timestep_spacing is supported");
    if (c.final_sigmas_type != "zero") throw std::invalid_argument("only zero final_sigmas_type is supported");
    if (c.num_train_timesteps == 0) throw std::invalid_argument("num_train_timesteps must be positive");
    const float T = static_cast<float>(c.num_train_timesteps);
    std::vector<float> shifted(n + 1);
    for (size_t i = 0; i <= n; ++i) {
        const float a = 1.0f + (1.0f / T - 1.0f) * (static_cast<float>(i) / static_cast<float>(n));
        const float s = 1.0f - a;
        shifted[i] = c.flow_shift * s / (1.0f + (c.flow_shift - 1.0f) * s);
    }
    SanaSchedulerTimesteps out;
    for (size_t i = 0; i < n; ++i) {
        const float s = shifted[n - i];
        out.sigmas.push_back(s);
        out.timesteps.push_back(static_cast<float>(static_cast<int>(s * T)));
    }
    out.sigmas.push_back(0.0f);
    return out;
}

SanaSchedulerState init_sana_scheduler_state(size_t n, const SanaSchedulerConfig & c) {
    check_config(c);
    SanaSchedulerState st;
    st.schedule = build_sana_scheduler_timesteps(n, c);
    return st;
}

Tensor convert_sana_scheduler_model_output(const Tensor & v, const Tensor & x, const SanaSchedulerState & st,
                                           const SanaSchedulerConfig & c) {
    check_config(c);
    check_step(st);
    if (!v.same_shape(x)) throw std::invalid_argument("model_output and sample must have the same shape");
    const float sigma = st.schedule.sigmas[st.step_index];
    Tensor out(x.shape());
    for (size_t i = 0; i < out.numel(); ++i) out.data()[i] = x.data()[i] - sigma * v.data()[i];
    return out;
}

Tensor sana_scheduler_first_order_update(const Tensor & x0, const Tensor & x, const SanaSchedulerState & st,
                                         const SanaSchedulerConfig & c) {
    check_config(c);
    check_step(st);
    if (!x0.same_shape(x)) throw std::invalid_argument("converted_model_output and sample must have the same shape");
    float at, st_, as, ss;
    alpha_sigma(st.schedule.sigmas[st.step_index + 1], c, at, st_);
    alpha_sigma(st.schedule.sigmas[st.step_index], c, as, ss);
    const float h = lambda_of(at, st_) - lambda_of(as, ss);
    const float ca = st_ / ss, cb = -at * (std::exp(-h) - 1.0f);
    Tensor out(x.shape());
    for (size_t i = 0; i < out.numel(); ++i) out.data()[i] = ca * x.data()[i] + cb * x0.data()[i];
    return out;
}

Tensor sana_scheduler_second_order_update(const Tensor & x, const SanaSchedulerState & st,
                                          const SanaSchedulerConfig & c) {
    check_config(c);
    check_step(st);
    if (st.step_index == 0) throw std::invalid_argument("second-order update requires at least one previous step");
    if (st.previous_model_outputs.size() < 2)
        throw std::invalid_argument("second-order update requires two model outputs");
    float at, sgt, a0, s0, a1, s1;
    alpha_sigma(st.schedule.sigmas[st.step_index + 1], c, at, sgt);
    alpha_sigma(st.schedule.sigmas[st.step_index], c, a0, s0);
    alpha_sigma(st.schedule.sigmas[st.step_index - 1], c, a1, s1);
    const float lt = lambda_of(at, sgt), l0 = lambda_of(a0, s0), l1 = lambda_of(a1, s1);
    const Tensor & m0 = st.previous_model_outputs.back();
    const Tensor & m1 = st.previous_model_outputs[st.previous_model_outputs.size() - 2];
    if (!m0.same_shape(x) || !m1.same_shape(x))
        throw std::invalid_argument("stored model outputs must match sample shape");
    const float h = lt - l0, r0 = (l0 - l1) / h;
    const float ca = sgt / s0, cb = -at * (std::exp(-h) - 1.0f);
    const float cc = c.solver_type == "midpoint" ? -0.5f * at * (std::exp(-h) - 1.0f)
                                                 : at * ((std::exp(-h) - 1.0f) / h + 1.0f);
    Tensor out(x.shape());
    for (size_t i = 0; i < out.numel(); ++i) {
        const float d1 = (1.0f / r0) * (m0.data()[i] - m1.data()[i]);
        out.data()[i] = ca * x.data()[i] + cb * m0.data()[i] + cc * d1;
    }
    return out;
}

Tensor step_sana_scheduler(const Tensor & v, const Tensor & x, SanaSchedulerState & st,
                           const SanaSchedulerConfig & c) {
    check_config(c);
    check_step(st);
    if (!v.same_shape(x)) throw std::invalid_argument("model_output and sample must have the same shape");
    Tensor x0 = convert_sana_scheduler_model_output(v, x, st, c);
    st.previous_model_outputs.push_back(x0);
    if (st.previous_model_outputs.size() > c.solver_order)
        st.previous_model_outputs.erase(st.previous_model_outputs.begin());
    const size_t n = st.schedule.timesteps.size();
    const bool final_first_order = st.step_index == n - 1 && (c.lower_order_final || c.final_sigmas_type == "zero");
    Tensor out = (c.solver_order == 1 || st.lower_order_step_count < 1 || final_first_order)
                     ? sana_scheduler_first_order_update(x0, x, st, c)
                     : sana_scheduler_second_order_update(x, st, c);
    if (st.lower_order_step_count < c.solver_order) st.lower_order_step_count += 1;
    st.step_index += 1;
    return out;
}
