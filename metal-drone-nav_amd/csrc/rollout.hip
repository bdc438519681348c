// rollout.hip — batched environment step + rollout actor/critic for gfx950.
//
// One persistent launch runs `count` ticks of Sim::collect (main.mm:573-598):
// per tick sim_depth, sim_observe, the actor forward, sim_act and
// sim_advance (sim.metal:145-332) of the reference, fused.  Environments are
// independent, so a workgroup never waits on another: each env is owned by a
// group of G lanes of one wave for the whole launch, its state and controller
// memory stay in registers, and its obstacles, pooled depth ring, observation
// row and hidden activations live in LDS.  The G lanes split the data-parallel
// parts (pooled ray blocks, hidden units, RAPTOR rows) and compute the serial
// RK4 chain redundantly.  Every dot product keeps the reference's sequential
// order, so results round exactly like the CPU oracle.
#include "nav_device.h"
#include "nav_episode.h"
#include "kernel_args.h"

namespace nav {



// ---------------------------------------------------------------- group helpers
// A lane group never straddles a wavefront (64 % G == 0), and LDS accesses of
// one wavefront are performed in program order, so ordering the group's LDS
// traffic only needs a wavefront-scope fence that the compiler cannot move
// accesses across.
__device__ __forceinline__ void group_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ float fbits(uint32_t u) { return bits_float(u); }
// lane Q of this lane's quad (DPP quad_perm [Q,Q,Q,Q])
template <int Q>
__device__ __forceinline__ float quad_bcast(float x) {
    return bits_float(uint32_t(__builtin_amdgcn_update_dpp(0, int(float_bits(x)), 0x55 * Q, 0xF, 0xF, false)));
}
__device__ __forceinline__ uint32_t ubits(float f) { return float_bits(f); }

// RAPTOR step over a group of G lanes (raptor.hpp:52-97): lane `lane` owns
// input rows and GRU units lane + G*j; the dense output and the clip are
// evaluated by every lane.  `hidden` is the full recurrent state (identical in
// all lanes), `hu` this lane's own units.  Two group barriers; call from
// uniform control flow with `on` masking inactive groups.
template <int G>
__device__ __forceinline__ void raptor_group(const float* RW, const float (&mo)[22], float (&hidden)[16],
                                             float (&hu)[16 / G], float* sx, float* sh, uint32_t lane, bool on,
                                             float (&act)[4]) {
    constexpr int U = 16 / G;
    if (on) {
#pragma unroll
        for (int j = 0; j < U; j++) {  // Dense 22->16 + ReLU (raptor.hpp:54-60)
            const uint32_t row16 = lane + G * j;
            float val = RW[352 + row16];
#pragma unroll
            for (int col = 0; col < 22; col++) val = fma_f(RW[row16 * 22 + col], mo[col], val);
            sx[row16] = max_f(val, 0.0f);
        }
    }
    group_sync();
    float nh[U];
    if (on) {
        float x[16];
#pragma unroll
        for (int col = 0; col < 16; col++) x[col] = sx[col];
#pragma unroll
        for (int j = 0; j < U; j++) {  // GRU (raptor.hpp:62-84): unit u uses rows u, 16+u, 32+u
            const uint32_t u = lane + G * j;
            float iv[3], hv[3];
#pragma unroll
            for (int g3 = 0; g3 < 3; g3++) {
                const uint32_t rowg = u + 16 * g3;
                float ivv = RW[1904 + rowg], hvv = RW[1952 + rowg];
#pragma unroll
                for (int col = 0; col < 16; col++) {
                    ivv = fma_f(RW[368 + rowg * 16 + col], x[col], ivv);
                    hvv = fma_f(RW[1136 + rowg * 16 + col], hidden[col], hvv);
                }
                iv[g3] = ivv;
                hv[g3] = hvv;
            }
            const float reset = sigmoid_f(iv[0] + hv[0]);
            const float update = sigmoid_f(iv[1] + hv[1]);
            const float cand = tanh_f(iv[2] + reset * hv[2]);
            nh[j] = (1.0f - update) * cand + update * hu[j];
            sh[u] = nh[j];
        }
    }
    group_sync();
    if (on) {
#pragma unroll
        for (int j = 0; j < U; j++) hu[j] = nh[j];
#pragma unroll
        for (int col = 0; col < 16; col++) hidden[col] = sh[col];
#pragma unroll
        for (int q = 0; q < 4; q++) {  // output dense + clip (raptor.hpp:86-97)
            float val = RW[2080 + q];
#pragma unroll
            for (int col = 0; col < 16; col++) val = fma_f(RW[2016 + q * 16 + col], hidden[col], val);
            act[q] = max_f(-1.0f, min_f(1.0f, val));
        }
    }
}

__device__ __forceinline__ bool clean_env(const MdnSimConfig& c, uint32_t n) {
    return c.eval == 0 && ((c.family == 12 || c.family == 13) && n % 2 == 0);  // sim.metal:17-21
}

__device__ __forceinline__ void load_state(const float* g, uint32_t N, uint32_t n, State& s) {
    float* d = &s.p[0];
#pragma unroll
    for (uint32_t i = 0; i < STATE_WORDS; i++) d[i] = g[size_t(i) * N + n];
}
__device__ __forceinline__ void store_state(float* g, uint32_t N, uint32_t n, const State& s, uint32_t lane, uint32_t G) {
    const float* d = &s.p[0];
#pragma unroll
    for (uint32_t i = 0; i < STATE_WORDS; i++)
        if (i % G == lane) g[size_t(i) * N + n] = d[i];
}
__device__ __forceinline__ void load_run(const uint32_t* g, uint32_t N, uint32_t n, Run& r) {
    uint32_t* d = reinterpret_cast<uint32_t*>(&r);
#pragma unroll
    for (uint32_t i = 0; i < RW_COUNT; i++) d[i] = g[size_t(i) * N + n];
}
__device__ __forceinline__ void store_run(uint32_t* g, uint32_t N, uint32_t n, const Run& r, uint32_t lane, uint32_t G) {
    const uint32_t* d = reinterpret_cast<const uint32_t*>(&r);
#pragma unroll
    for (uint32_t i = 0; i < RW_COUNT; i++)
        if (i % G == lane) g[size_t(i) * N + n] = d[i];
}

// Reset bookkeeping shared by the first reset and the auto-reset
// (sim.metal:55-94 == cpu_reference.hpp:240-273): returns the episode
// family and world seed drawn from the env's RNG.
__device__ __forceinline__ void reset_draw(const MdnSimConfig& c, uint32_t n, bool first, uint32_t& rng,
                                           uint32_t& family, uint32_t& world_seed) {
    rng = first ? c.seed + n * 747796405u + 2891336453u : rng;
    family = c.family == MDN_FAMILY_C3_MIX ? MDN_C3_LANE_FAMILY(n) : training_family(c.family, rng);
    world_seed = xs(rng);
}

// After the world is generated: wind, start pose, hover rpm, controller
// memory, episode counters.
__device__ __forceinline__ void reset_apply(const MdnSimConfig& c, const MdnPhysicsParams& P, const float* raptor,
                                            uint32_t n, bool first, uint32_t rng, float* world, State& s, Run& r) {
    world[166] = clean_env(c, n) ? 0.0f : c.wind;
    world[167] = 0;
    world[168] = 0;
#pragma unroll
    for (int j = 0; j < 3; j++) {
        s.p[j] = j == 2 ? 1.5f : 0;
        s.v[j] = 0;
        s.w[j] = 0;
        r.desired_vel[j] = 0;
        r.ref_pos[j] = s.p[j];
    }
    s.q[0] = 1; s.q[1] = 0; s.q[2] = 0; s.q[3] = 0;
    const float target = P.mass * 9.81f / 4;
    const float c0 = P.rotor_thrust_coefficients[0], c1 = P.rotor_thrust_coefficients[1], c2 = P.rotor_thrust_coefficients[2];
    const float hover = clamp_f((-c1 + sqrt_f(c1 * c1 - 4 * c2 * (c0 - target))) / (2 * c2), P.action_min, P.action_max);
#pragma unroll
    for (int j = 0; j < 16; j++) r.hidden[j] = raptor[2000 + j];
#pragma unroll
    for (int j = 0; j < 4; j++) { s.rpm[j] = hover; r.motors[j] = 0; r.prev_nav[j] = 0; }
    const uint32_t wfam = float_bits(world[162]);
    if (wfam == 10 || wfam == 11) {
        s.v[0] = c.speed;
        r.desired_vel[0] = c.speed;
        r.prev_nav[0] = 1.0f;
    }
    r.yaw = 0; r.rng = rng; r.steps = 0; r.path = 0; r.elapsed = 0; r.peak_speed = 0;
    r.min_clearance = 12;
    const float gx = world[163], gy = world[164], gz = world[165] - 1.5f;
    r.initial_distance = sqrt_f(gx * gx + gy * gy + gz * gz);
    if (first) {
        r.successes = r.collisions = r.timeouts = r.episodes = 0;
        r.success_time = r.total_path = r.total_elapsed = r.final_progress = 0;
    }
}

// First reset of every env (sim_reset kernel, sim.metal:142-144): one
// thread per env, writes straight to the global buffers.
__global__ __launch_bounds__(64) void reset_kernel(RolloutArgs a) {
    const uint32_t n = blockIdx.x * 64 + threadIdx.x;
    const uint32_t N = a.cfg.n;
    if (n >= N) return;
    State s;
    Run r;
    load_run(a.run, N, n, r);
    uint32_t rng = 0, family = 0, seed = 0;
    reset_draw(a.cfg, n, true, rng, family, seed);
    float* world = a.world + size_t(n) * WORLD_WORDS;
    WorldGen wg{world};
    wg.generate(seed, family, a.cfg.distance);
    reset_apply(a.cfg, a.phys, a.raptor, n, true, rng, world, s, r);
    store_state(a.state, N, n, s, 0, 1);
    store_run(a.run, N, n, r, 0, 1);
    for (uint32_t j = 0; j < 8 * PIX; j++) a.sensors[size_t(n) * 8 * PIX + j] = 12.0f;
    for (uint32_t j = 0; j < 32; j++) a.commands[size_t(n) * 32 + j] = 0.0f;
    for (uint32_t j = 0; j < 96; j++) a.poses[size_t(n) * 96 + j] = 0.0f;
}

// Per-episode work of the envs whose episode just began, one thread per env:
// the episode's plant (sim.metal:62-69, with its hover rpm 70-81), its
// challenge-bank world (sim.metal:95-121) and its navigation task
// (sim.metal:122-141: world, start state, yaw, reference point, desired
// velocity, initial distance, wind), in the reference's order.  Runs after the reset
// kernel (first: every env) and after each launch that may reset envs (an
// env with steps == 0 was reset by it; an evaluation never restarts one).
// One wavefront per env: every lane computes the same values (and stores
// the same words), except the task generator's segment clearances, whose
// samples the lanes share.  The workgroup is that one wavefront, so the
// plant, its draw, the task state and the witness path live in its LDS.
__global__ __launch_bounds__(64) void episode_kernel(EpisodeArgs a) {
    const uint32_t n = blockIdx.x;
    const uint32_t N = a.cfg.n;
    if (n >= N) return;  // uniform over the wavefront
    Run r;
    load_run(a.run, N, n, r);
    if (!a.first && r.steps != 0u) return;
    State s;
    load_state(a.state, N, n, s);
    // the plant and its draw live in the wavefront's LDS (88 words each, the
    // same values from every lane), not in registers
    __shared__ MdnPhysicsParams s_ep, s_varied;
    MdnPhysicsParams& ep = s_ep;
    ep = a.phys;
    if (a.runtime.enabled != 0u && a.runtime.domain_amplitude > 0.0f) {
        const uint32_t rng = dom_seed(a.runtime, a.cfg.seed, n, a.first ? 0u : r.episodes);
        if (dom_sample(a.phys, rng, a.runtime.domain_amplitude, a.runtime.domain_range, s_varied)) ep = s_varied;
        else ep.mass = nan_f();  // rejected draw: the host's validation reports it
    }
    a.env_phys[n] = ep;
    if (a.runtime.enabled != 0u) {
        const float target = ep.mass * 9.81f / 4;
        for (int q = 0; q < 4; q++) {
            const float c0 = ep.rotor_thrust_coefficients[3 * q], c1 = ep.rotor_thrust_coefficients[3 * q + 1],
                        c2 = ep.rotor_thrust_coefficients[3 * q + 2];
            const float disc = c1 * c1 - 4 * c2 * (c0 - target);
            s.rpm[q] = disc >= 0.0f ? clamp_f((-c1 + sqrt_f(disc)) / (2 * c2), ep.action_min, ep.action_max)
                                    : ep.action_max;
        }
    }
    float* world = a.world + size_t(n) * WORLD_WORDS;
    if (a.bank.enabled != 0u) {  // sim.metal:95-121
        if (a.bank.bank_count != 0u && a.slot < a.bank.schedule_stride) {
            const uint32_t level = a.bank_schedule[size_t(n) * a.bank.schedule_stride + a.slot];
            bool apply = true;
            if (level == MDN_BANK_REHEARSAL) {  // alternating static / moving-threat rehearsal
                uint32_t rng = r.rng;
                const uint32_t family = training_family(n % 2 == 0 ? 12u : 13u, rng);
                const uint32_t seed = xs(rng);
                WorldGen{world}.generate(seed, family, 4.0f);
                r.rng = rng;
            } else if (level < a.bank.bank_count) {
                const float* src = a.bank_worlds + size_t(level) * WORLD_WORDS;
                for (uint32_t i = 0; i < WORLD_WORDS; i++) world[i] = src[i];
            } else {
                apply = false;
            }
            if (apply) {
                world[166] = clean_env(a.cfg, n) ? 0.0f : a.cfg.wind;
                world[167] = 0.0f;
                world[168] = 0.0f;
                const float gx = world[163], gy = world[164], gz = world[165] - 1.5f;
                r.initial_distance = sqrt_f(gx * gx + gy * gy + gz * gz);
                const uint32_t wfam = float_bits(world[162]);
                if (wfam == 10u || wfam == 11u) {
                    s.v[0] = a.cfg.speed;
                    r.desired_vel[0] = a.cfg.speed;
                    r.prev_nav[0] = 1.0f;
                }
                a.bank_active[n] = level;
            }
        }
    } else {
        a.bank_active[n] = MDN_BANK_REHEARSAL;
    }
    __shared__ MdnTaskState s_task;  // in LDS like the plant
    MdnTaskState& t = s_task;
    uint32_t* tw = reinterpret_cast<uint32_t*>(&t);
    for (uint32_t i = 0; i < sizeof(MdnTaskState) / 4; i++) tw[i] = 0u;
    if (a.task.enabled != 0u) {
        uint32_t rng = a.cfg.seed ^ ((n + 1u) * 0x27d4eb2du) ^ ((r.episodes + 1u) * 0x165667b1u);
        task_generate(world, t, rng, a.task.config);
        if (t.valid != 0u) {
#pragma unroll
            for (int k = 0; k < 3; k++) {
                s.p[k] = t.start_position[k];
                s.v[k] = t.start_velocity_world[k];
                s.w[k] = 0.0f;
            }
            float sh, ch;
            sincos_f(t.start_yaw_rad * 0.5f, &sh, &ch);
            s.q[0] = ch; s.q[1] = 0.0f; s.q[2] = 0.0f; s.q[3] = sh;
            r.yaw = t.start_yaw_rad;
            r.initial_distance = t.initial_distance_m;
#pragma unroll
            for (int k = 0; k < 3; k++) {
                r.ref_pos[k] = s.p[k];
                r.desired_vel[k] = s.v[k];
            }
            world[166] = clean_env(a.cfg, n) ? 0.0f : a.cfg.wind;
            world[167] = 0.0f;
            world[168] = 0.0f;
        }
    }
    a.task_states[n] = t;
    store_state(a.state, N, n, s, 0, 1);
    store_run(a.run, N, n, r, 0, 1);
}

// ---------------------------------------------------------------- matrix-core layer
// One hidden layer for 32 envs on the fp32 matrix cores: out[env][unit] =
// tanh(b1[unit] + sum_k x[env][k] * w1t[k][unit]).  v_mfma_f32_16x16x4_f32
// applies acc = fma(a[k], b[k], acc) for its four k in ascending order with
// one rounding each, so the chain over k0 = 0, 4, 8, ... is exactly the
// canonical fma chain from the bias.  A lane a holds A[a%16][k0 + a/16], B
// lane a holds B[k0 + a/16][a%16], accumulator r of lane l is
// D[4(l/16) + r][l%16].  Wavefront w computes tiles 2w and 2w+1 of the 2 x 4
// grid of 16x16 tiles (env block = tile / 4, unit block = tile % 4).
typedef float v4f __attribute__((ext_vector_type(4)));
// The operands of k-step s are read from LDS PF steps before its MFMAs issue
// (a scheduling fence between steps keeps that order), so the LDS latency of
// one step overlaps the matrix-core work of the previous ones.
constexpr uint32_t MFMA_PF = 3;
template <uint32_t D, uint32_t XS, uint32_t OS>
__device__ __forceinline__ void wg_layer(const float* x, const float* w1t, const float* b1, float* out) {
    const uint32_t wv = threadIdx.x / 64, l = threadIdx.x % 64;
    // tiles 2w and 2w+1 share env block w/2: one A operand for both
    const uint32_t env = 16 * (wv / 2) + l % 16;
    uint32_t unit[2];
    v4f acc[2];
#pragma unroll
    for (uint32_t q = 0; q < 2; q++) {
        unit[q] = 16 * ((2 * wv + q) % 4) + l % 16;
        const float bias = b1[unit[q]];
        acc[q][0] = bias; acc[q][1] = bias; acc[q][2] = bias; acc[q][3] = bias;
    }
    constexpr uint32_t NK = (D + 3) / 4;
    float av[NK], bv[NK][2];
#pragma unroll
    for (uint32_t st = 0; st < NK + MFMA_PF; st++) {
        if (st < NK) {
            const uint32_t k = 4 * st + l / 16;
            av[st] = k < D ? x[env * XS + k] : 0.0f;
#pragma unroll
            for (uint32_t q = 0; q < 2; q++) bv[st][q] = k < D ? w1t[k * HID + unit[q]] : -0.0f;
        }
        if (st >= MFMA_PF) {
            const uint32_t u = st - MFMA_PF;
#pragma unroll
            for (uint32_t q = 0; q < 2; q++) acc[q] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[u], bv[u][q], acc[q], 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    const uint32_t e0 = env - l % 16 + 4 * (l / 16);
#pragma unroll
    for (uint32_t q = 0; q < 2; q++)
#pragma unroll
        for (uint32_t r = 0; r < 4; r++) out[(e0 + r) * OS + unit[q]] = tanh_f(acc[q][r]);
}

// wg_layer with the weight operands already in registers: bw[q][kk] is
// w1t[4 kk + l/16][unit of tile q] for lane l (see critic_operands).
template <uint32_t D, uint32_t XS, uint32_t OS>
__device__ __forceinline__ void wg_layer_rb(const float* x, const float (&bw)[2][D / 4], const float* b1, float* out) {
    static_assert(D % 4 == 0, "whole k-steps");
    const uint32_t wv = threadIdx.x / 64, l = threadIdx.x % 64;
    const uint32_t env = 16 * (wv / 2) + l % 16;
    uint32_t unit[2];
    v4f acc[2];
#pragma unroll
    for (uint32_t q = 0; q < 2; q++) {
        unit[q] = 16 * ((2 * wv + q) % 4) + l % 16;
        const float bias = b1[unit[q]];
        acc[q][0] = bias; acc[q][1] = bias; acc[q][2] = bias; acc[q][3] = bias;
    }
    constexpr uint32_t NK = D / 4;
    float av[NK];
#pragma unroll
    for (uint32_t st = 0; st < NK + MFMA_PF; st++) {
        if (st < NK) av[st] = x[env * XS + 4 * st + l / 16];
        if (st >= MFMA_PF) {
            const uint32_t u = st - MFMA_PF;
#pragma unroll
            for (uint32_t q = 0; q < 2; q++) acc[q] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[u], bw[q][u], acc[q], 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    const uint32_t e0 = env - l % 16 + 4 * (l / 16);
#pragma unroll
    for (uint32_t q = 0; q < 2; q++)
#pragma unroll
        for (uint32_t r = 0; r < 4; r++) out[(e0 + r) * OS + unit[q]] = tanh_f(acc[q][r]);
}
// This lane's weight operands of wg_layer_rb for w1t[D][HID].
template <uint32_t D>
__device__ __forceinline__ void critic_operands(const float* w1t, float (&bw)[2][D / 4]) {
    const uint32_t wv = threadIdx.x / 64, l = threadIdx.x % 64;
#pragma unroll
    for (uint32_t q = 0; q < 2; q++) {
        const uint32_t unit = 16 * ((2 * wv + q) % 4) + l % 16;
#pragma unroll
        for (uint32_t kk = 0; kk < D / 4; kk++) bw[q][kk] = w1t[(4 * kk + l / 16) * HID + unit];
    }
}

// Output heads for the 32 envs of a workgroup on the matrix cores:
// out[env * 17 + c] = b[c] + sum_h w[c][h] * x[env][h] (c < NC), the fma chain
// over the 64 hidden units ascending from the bias, as a 16x16x4 tile per
// env block (columns c >= NC multiply by -0.0 and are not stored).  Wavefronts
// w0 and w0+1 compute env blocks 0 and 1; `wstride` is the row stride of w.
template <uint32_t NC, uint32_t XS>
__device__ __forceinline__ void wg_head(const float* x, const float* w, uint32_t wstride, const float* b, uint32_t w0,
                                        float* out, uint32_t col0) {
    const uint32_t wv = threadIdx.x / 64, l = threadIdx.x % 64, c = l % 16;
    if (wv < w0 || wv >= w0 + 2) return;
    const uint32_t eb = wv - w0, env = 16 * eb + c;
    v4f acc;
    const float bias = c < NC ? b[c] : 0.0f;
    acc[0] = bias; acc[1] = bias; acc[2] = bias; acc[3] = bias;
    constexpr uint32_t NK = HID / 4;
    float av[NK], bv[NK];
#pragma unroll
    for (uint32_t st = 0; st < NK + MFMA_PF; st++) {
        if (st < NK) {
            const uint32_t k = 4 * st + l / 16;
            av[st] = x[env * XS + k];
            bv[st] = c < NC ? w[c * wstride + k] : -0.0f;
        }
        if (st >= MFMA_PF) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[st - MFMA_PF], bv[st - MFMA_PF], acc, 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
    }
    if (c < NC)
#pragma unroll
        for (uint32_t r = 0; r < 4; r++) out[(16 * eb + 4 * (l / 16) + r) * 17 + col0 + c] = acc[r];
}

// Lane-constant RAPTOR operands of raptor_wave, read once per launch: the
// B operands of the dense layer (dense[kk] = W[j][4 kk + kq]) and of the GRU
// gate products (gi/gh[g][kk] = W_ih/W_hh[16 g + j][4 kk + kq]), and the
// output layer as an A operand (out[kk] = W_out[j][4 kk + kq], rows j >= 4
// zero) with its bias in the accumulator rows this lane holds (lane l, kq =
// l / 16, j = l % 16).
struct RaptorRegs {
    float dense[6], gi[3][4], gh[3][4], out[4], obias[4];
};
__device__ __forceinline__ void raptor_operands(const float* RW, RaptorRegs& o) {
    const uint32_t l = threadIdx.x % 64, j = l % 16, kq = l / 16;
#pragma unroll
    for (uint32_t kk = 0; kk < 6; kk++) {
        const uint32_t k = 4 * kk + kq;
        o.dense[kk] = k < 22 ? RW[j * 22 + k] : -0.0f;
    }
#pragma unroll
    for (uint32_t g = 0; g < 3; g++)
#pragma unroll
        for (uint32_t kk = 0; kk < 4; kk++) {
            o.gi[g][kk] = RW[368 + (16 * g + j) * 16 + 4 * kk + kq];
            o.gh[g][kk] = RW[1136 + (16 * g + j) * 16 + 4 * kk + kq];
        }
#pragma unroll
    for (uint32_t kk = 0; kk < 4; kk++) o.out[kk] = j < 4 ? RW[2016 + j * 16 + 4 * kk + kq] : 0.0f;
#pragma unroll
    for (uint32_t r = 0; r < 4; r++) o.obias[r] = kq == 0 ? RW[2080 + r] : 0.0f;
}

// RAPTOR step (raptor.hpp:52-97) for the 8 envs of one wavefront on the
// matrix cores, with no workgroup barrier: 16x16x4 tiles whose fma chains
// run from the biases over the inputs in ascending order (the chain of
// raptor_group), tile row i holding the wavefront's env i % 8 (rows 8-15
// repeat rows 0-7).  The GRU's input-side and hidden-side
// products land in the same lanes, so each lane evaluates the gates of two
// (env, unit) pairs from registers.  The output layer is the product
// W_out . h^T (outputs as rows, envs as columns), its chain over the 16
// hidden units ascending from the bias; lane e < 8 then holds env e's four
// outputs and each group reads them from there.  `smo` holds the group's
// observation row (stride MS), `sx` the dense output, `srh` the hidden state
// (stride 17).  Call from uniform control flow; `on` masks envs whose step
// is skipped.
template <int G, uint32_t MS>
__device__ __forceinline__ void raptor_wave(const float* RW, const RaptorRegs& o, const float (&mo)[22], float* smo,
                                            float* sx, float* srh, uint32_t grp, uint32_t lane, bool on,
                                            float (&act)[4]) {
    static_assert(G == 8, "one tile row per env: 8 envs per wavefront");
    const uint32_t l = threadIdx.x % 64, j = l % 16, kq = l / 16;
    const uint32_t base = (threadIdx.x / 64) * 8, env = base + j % 8;
#pragma unroll
    for (int c = 0; c < 22; c++) smo[grp * MS + c] = mo[c];  // equal values from the group's lanes
    group_sync();
    {   // Dense 22->16 + ReLU (raptor.hpp:54-60)
        v4f acc;
        const float bias = RW[352 + j];
        acc[0] = bias; acc[1] = bias; acc[2] = bias; acc[3] = bias;
        float av[6];
#pragma unroll
        for (uint32_t kk = 0; kk < 6; kk++) {
            const uint32_t k = 4 * kk + kq;
            av[kk] = k < 22 ? smo[env * MS + k] : 0.0f;
        }
#pragma unroll
        for (uint32_t kk = 0; kk < 6; kk++) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[kk], o.dense[kk], acc, 0, 0, 0);
        if (kq < 2)
#pragma unroll
            for (uint32_t r = 0; r < 4; r++) sx[(base + 4 * kq + r) * 17 + j] = max_f(acc[r], 0.0f);
    }
    group_sync();
    // GRU gate products (raptor.hpp:62-84): gate g of unit u is row 16g + u.
    // Lane (kq, j) holds envs 4 kq + r (mod 8) of unit j; lanes kq < 2 keep
    // rows r = 0, 1 and lanes kq >= 2 rows 2, 3, so each env is taken once.
    const bool lo = kq < 2;
    float ax[4], ah[4];
#pragma unroll
    for (uint32_t kk = 0; kk < 4; kk++) {
        ax[kk] = sx[env * 17 + 4 * kk + kq];
        ah[kk] = srh[env * 17 + 4 * kk + kq];
    }
    // one gate at a time (two chains live), each folded into the gate
    // values as soon as it is complete
    float reset[2], update[2], nh[2], hold[2];
    uint32_t e2[2];
#pragma unroll
    for (uint32_t p = 0; p < 2; p++) {
        e2[p] = base + (4 * kq + (lo ? p : 2 + p)) % 8;
        hold[p] = srh[e2[p] * 17 + j];
    }
#pragma unroll
    for (uint32_t g = 0; g < 3; g++) {
        v4f ci, ch;
        const float bi = RW[1904 + 16 * g + j], bh = RW[1952 + 16 * g + j];
        ci[0] = bi; ci[1] = bi; ci[2] = bi; ci[3] = bi;
        ch[0] = bh; ch[1] = bh; ch[2] = bh; ch[3] = bh;
#pragma unroll
        for (uint32_t kk = 0; kk < 4; kk++) {
            ci = __builtin_amdgcn_mfma_f32_16x16x4f32(ax[kk], o.gi[g][kk], ci, 0, 0, 0);
            ch = __builtin_amdgcn_mfma_f32_16x16x4f32(ah[kk], o.gh[g][kk], ch, 0, 0, 0);
        }
#pragma unroll
        for (uint32_t p = 0; p < 2; p++) {
            // rows p and 2 + p as two fixed registers and one select each (an
            // empty asm keeps the compiler from turning the pair into a
            // lane-dependent row index, which it expands to a compare chain)
            float i0 = ci[p], i2 = ci[2 + p], h0 = ch[p], h2 = ch[2 + p];
            asm volatile("" : "+v"(i0), "+v"(i2), "+v"(h0), "+v"(h2));
            const float iv = lo ? i0 : i2, hv = lo ? h0 : h2;
            if (g == 0) {
                reset[p] = sigmoid_f(iv + hv);
            } else if (g == 1) {
                update[p] = sigmoid_f(iv + hv);
            } else {
                const float cand = tanh_f(iv + reset[p] * hv);
                nh[p] = (1.0f - update[p]) * cand + update[p] * hold[p];
            }
        }
    }
    const uint64_t live = __ballot(on);
    bool on2[2];
#pragma unroll
    for (uint32_t p = 0; p < 2; p++) on2[p] = (live >> ((e2[p] - base) * G)) & 1ull;
    group_sync();  // every lane's reads of the old hidden state precede the writes
#pragma unroll
    for (uint32_t p = 0; p < 2; p++)
        if (on2[p]) srh[e2[p] * 17 + j] = nh[p];
    group_sync();
    {   // output dense + clip (raptor.hpp:86-97)
        v4f acc;
#pragma unroll
        for (uint32_t r = 0; r < 4; r++) acc[r] = o.obias[r];
        float bh[4];
#pragma unroll
        for (uint32_t kk = 0; kk < 4; kk++) bh[kk] = srh[env * 17 + 4 * kk + kq];
#pragma unroll
        for (uint32_t kk = 0; kk < 4; kk++) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(o.out[kk], bh[kk], acc, 0, 0, 0);
        const int src = int((threadIdx.x % 64) / G);  // lane holding this group's env column
#pragma unroll
        for (uint32_t q = 0; q < 4; q++) act[q] = __builtin_amdgcn_fmed3f(__shfl(acc[q], src, 64), -1.0f, 1.0f);
    }
}

// ---------------------------------------------------------------- rollout
// W = wavefronts per workgroup.  W == 1: weights and camera rays are read from
// global memory (L1/L2 resident).  W > 1: the workgroup stages one copy of the
// actor first layer, the RAPTOR weights and the camera rays in LDS, shared by
// its 64*W/G envs.
// Tails of the flat policy vectors (ppo.hpp:35-45) from the first bias on:
// actor b1[HID], W2[4][HID], b2[4], log_std[4]; critic b1[HID], W2[HID], b2.
constexpr uint32_t ACTOR_TAIL = 5 * HID + 8, CRITIC_TAIL = 2 * HID + 1;

// Stages NW consecutive words into LDS with the workgroup's NTH threads:
// every thread's loads are issued before its first store (fixed trip count).
template <uint32_t NW, uint32_t NTH>
struct WordStage {
    static constexpr uint32_t R = (NW + NTH - 1) / NTH;
    float v[R];
    __device__ __forceinline__ void load(const float* __restrict__ src, uint32_t t) {
#pragma unroll
        for (uint32_t j = 0; j < R; j++) {
            const uint32_t i = t + NTH * j;
            v[j] = src[i < NW ? i : 0];
        }
    }
    __device__ __forceinline__ void store(float* dst, uint32_t t) const {
#pragma unroll
        for (uint32_t j = 0; j < R; j++)
            if (t + NTH * j < NW) dst[t + NTH * j] = v[j];
    }
};
template <int W, uint32_t D>
struct WeightLds {
    float aw[D * HID];
    float rw[RAPTOR_WORDS];
    float cam[3 * PIX];
    float pol[ACTOR_TAIL + CRITIC_TAIL + 8];  // + exp(log_std), exp(-log_std)
};
template <uint32_t D>
struct WeightLds<1, D> {};

// X: split ticks. The kernel stops at the policy call and takes the means
// from a.ext_means (a policy evaluated by other kernels between launches);
// values and next values are the caller's.  D: actor inputs, 181 (pooled
// observation) or 184 (with the geometry-prior hint, ppo.hpp:30-34).
// DYN: per-episode plants (a.env_phys) and navigation tasks (a.task_cfg);
// launched one tick at a time around the episode kernel.
// CF: the launch's plant is the Crazyflie profile (checked byte for byte on
// the host), read as compile-time constants instead of from LDS.
template <int G, int K, int W, bool X, uint32_t D, bool DYN, bool CF = false>
__global__ __launch_bounds__(64 * W) void rollout_kernel(RolloutArgs a) {
    constexpr int E = 64 * W / G;    // envs per workgroup
    constexpr int U = 16 / G;        // RAPTOR units per lane
    constexpr int HU = 64 / G;       // actor/critic hidden units per lane
    const MdnSimConfig& C = a.cfg;
    __shared__ MdnPhysicsParams s_phys;
    if constexpr (!CF)
        for (uint32_t i = threadIdx.x; i < sizeof(MdnPhysicsParams) / 4; i += 64 * W)
            reinterpret_cast<float*>(&s_phys)[i] = reinterpret_cast<const float*>(&a.phys)[i];
    __syncthreads();
    const MdnPhysicsParams& P = plant_ref<CF>(s_phys);
    PhysRecip RP = kCrazyflieRecip;
    if constexpr (!CF) {
        RP.mass = a.recip_mass;
#pragma unroll
        for (int i = 0; i < 4; i++) { RP.rise[i] = a.recip_rise[i]; RP.fall[i] = a.recip_fall[i]; }
    }
    const uint32_t N = C.n;
    const uint32_t lane = threadIdx.x % G, grp = threadIdx.x / G;
    const uint32_t n = blockIdx.x * E + grp;
    const bool live = n < N;
    const uint32_t nn = live ? n : 0;

    constexpr uint32_t OS = D % 2 ? D + 4 : D + 3;  // odd stride of the observation rows
    // split ticks: the wide actor's loop and the 184-input actor's geometry
    // memory; the fused 181-input kernels keep the plain tick loop
    constexpr bool SPLIT = X || D == MDN_ACTOR_OBS_PRIOR || DYN;
    constexpr uint32_t WSTR = WORLD_WORDS;  // odd: env rows start in distinct banks
    // the env's state, counters, world and command rows are requested first,
    // so that their latency overlaps the shared weights' staging (a
    // split-tick launch pays this prologue once per tick)
    State s;
    Run r;
    load_state(a.state, N, nn, s);
    load_run(a.run, N, nn, r);
    constexpr uint32_t WR = (WORLD_WORDS + G - 1) / G, CMR = (32 + G - 1) / G;
    float wv[WR], cv[CMR];
#pragma unroll
    for (uint32_t j = 0; j < WR; j++) {
        const uint32_t i = lane + G * j;
        wv[j] = a.world[size_t(nn) * WORLD_WORDS + (i < WORLD_WORDS ? i : 0)];
    }
#pragma unroll
    for (uint32_t j = 0; j < CMR; j++) {
        const uint32_t i = lane + G * j;
        cv[j] = a.commands[size_t(nn) * 32 + (i < 32 ? i : 0)];
    }
    __shared__ WeightLds<W, D> s_wt;
    const float* AW1;   // actor W1 transposed [input][hidden]
    const float* RW;    // RAPTOR weights (RaptorWeights layout)
    const float* CAM;   // camera rays [pixel][3]
    if constexpr (W > 1) {
        // (unrolled: a split-tick launch stages the weights once per tick,
        // so their loads are kept in flight together)
        if constexpr (!X) {
#pragma unroll 8
            for (uint32_t i = threadIdx.x; i < D * HID; i += 64 * W) s_wt.aw[i] = a.actor_w1t[i];
        }
        WordStage<RAPTOR_WORDS, 64 * W> st_rw;
        WordStage<3 * PIX, 64 * W> st_cam;
        WordStage<ACTOR_TAIL, 64 * W> st_at;
        WordStage<CRITIC_TAIL, 64 * W> st_ct;
        st_rw.load(a.raptor, threadIdx.x);
        st_cam.load(a.camera, threadIdx.x);
        if constexpr (!X) st_at.load(a.actor + HID * D, threadIdx.x);
        st_ct.load(a.critic + HID * COBS, threadIdx.x);
        st_rw.store(s_wt.rw, threadIdx.x);
        st_cam.store(s_wt.cam, threadIdx.x);
        if constexpr (!X) st_at.store(s_wt.pol, threadIdx.x);
        st_ct.store(s_wt.pol + ACTOR_TAIL, threadIdx.x);
        __syncthreads();
        if constexpr (!X) {  // the action noise scales are fixed for the launch
            if (threadIdx.x < 8) {
                const float ls = s_wt.pol[5 * HID + 4 + threadIdx.x % 4];
                s_wt.pol[ACTOR_TAIL + CRITIC_TAIL + threadIdx.x] = exp_f(threadIdx.x < 4 ? ls : -ls);
            }
            __syncthreads();
        }
        AW1 = s_wt.aw;
        RW = s_wt.rw;
        CAM = s_wt.cam;
    } else {
        AW1 = a.actor_w1t;
        RW = a.raptor;
        CAM = a.camera;
    }

    __shared__ float s_world[E][WSTR];
    // Per-env rows have odd word strides so that the E groups of a wavefront,
    // reading the same offset of their own rows, fall in distinct banks.
    __shared__ float s_cent[E][49];
    // Pooled ring: slot j of the group's env at pring(g)[j * POOL].  In LDS,
    // except for the four-wavefront kernels with more than two slots, whose
    // LDS has no room for it: theirs is the env's row of a.pool_ring (read
    // back by the wavefront that wrote it, in program order).
    constexpr bool RING_HBM = W > 1 && K > 2;
    __shared__ float s_ring[E][RING_HBM ? 1 : K * POOL + 1];
    auto pring = [&](uint32_t g) -> float* {
        if constexpr (RING_HBM) {
            const uint32_t ng = blockIdx.x * E + g;
            return a.pool_ring + size_t(ng < N ? ng : 0) * K * POOL;
        } else {
            return s_ring[g];
        }
    };
    __shared__ float s_obs[E][OS];
    __shared__ float s_co[E][COBS + 1];
    __shared__ float s_ah[E][HID + 1];
    __shared__ float s_ch[E][HID + 1];
    __shared__ float s_cmd[E][33];
    __shared__ float s_x[E][17];
    __shared__ float s_h[W > 1 ? 1 : E][17];  // W == 1: the group step's new hidden state
    // W > 1: RAPTOR hidden state of each env, resident in LDS for the launch
    __shared__ float s_rh[W > 1 ? E : 1][17];

    float* world = s_world[grp];
#pragma unroll
    for (uint32_t j = 0; j < WR; j++)
        if (lane + G * j < WORLD_WORDS) world[lane + G * j] = wv[j];
#pragma unroll
    for (uint32_t j = 0; j < CMR; j++)
        if (lane + G * j < 32) s_cmd[grp][lane + G * j] = cv[j];
    {   // pooled ring cache: LDS slot f%K holds frame f for the last K frames
        // (a launch that begins at act already holds the frame cast for the
        // current step, if one was due); the 2x2 minima of the group's
        // K * POOL cells, ten cells' loads per lane in flight per round
        const int last = (SPLIT && (a.split & SPLIT_BEGIN_AT_ACT)) ? int(r.steps / C.sensor_period)
                         : r.steps == 0                         ? -1
                                                                : int((r.steps - 1) / C.sensor_period);
        constexpr uint32_t RC = (uint32_t(K) * POOL + G - 1) / G, CH = 10;  // cells per lane; per round
        for (uint32_t c0 = 0; c0 < RC; c0 += CH) {
            float px[CH][4];
#pragma unroll
            for (uint32_t c = 0; c < CH; c++) {
                const uint32_t e0 = lane + G * (c0 + c), e = e0 < uint32_t(K) * POOL ? e0 : 0;
                const int j = int(e / POOL), b = int(e % POOL);
                const int f = last - j;
                const uint32_t slot8 = uint32_t(((f % 8) + 8) % 8);
                const float* src = a.sensors + (size_t(nn) * 8 + slot8) * PIX;
                const uint32_t y = (b / 10) * 2, x = (b % 10) * 2;
#pragma unroll
                for (uint32_t dy = 0; dy < 2; dy++)
#pragma unroll
                    for (uint32_t dx = 0; dx < 2; dx++) px[c][2 * dy + dx] = src[(y + dy) * 20 + x + dx];
            }
#pragma unroll
            for (uint32_t c = 0; c < CH; c++) {
                const uint32_t e = lane + G * (c0 + c);
                if (e >= uint32_t(K) * POOL) continue;
                const int j = int(e / POOL), b = int(e % POOL);
                const int f = last - j;
                const uint32_t slotk = uint32_t(((f % K) + K) % K);
                float m = 12.0f;
#pragma unroll
                for (uint32_t q = 0; q < 4; q++) m = min_f(m, px[c][q]);
                if (live) pring(grp)[slotk * POOL + b] = m;
            }
        }
    }
    // this lane's RAPTOR units (hidden values it owns)
    float hu[U];
#pragma unroll
    for (int j = 0; j < U; j++) hu[j] = bits_float(a.run[size_t(RW_HIDDEN + lane + G * j) * N + nn]);
    if constexpr (W > 1) {
        constexpr uint32_t HR = (16 + G - 1) / G;
        float hv[HR];
#pragma unroll
        for (uint32_t j = 0; j < HR; j++) {
            const uint32_t c = lane + G * j;
            hv[j] = bits_float(a.run[size_t(RW_HIDDEN + (c < 16 ? c : 0)) * N + nn]);
        }
#pragma unroll
        for (uint32_t j = 0; j < HR; j++)
            if (lane + G * j < 16) s_rh[grp][lane + G * j] = hv[j];
    }
    const float* A = a.actor;
    const float* CR = a.critic;
    const uint32_t a_b1 = HID * D, a_w2 = a_b1 + HID, a_b2 = a_w2 + 4 * HID;
    const uint32_t c_b1 = HID * COBS, c_w2 = c_b1 + HID, c_b2 = c_w2 + HID;
    // W > 1: the policy tails from LDS and the critic's first layer in
    // registers (the tick loop then reads no weights from global memory)
    float cw1[2][COBS / 4];
    if constexpr (W > 1) critic_operands<COBS>(a.critic_w1t, cw1);
    RaptorRegs rops;
    if constexpr (W > 1) raptor_operands(RW, rops);
    const float* AT = A + a_b1;
    const float* CT = CR + c_b1;
    if constexpr (W > 1) {
        AT = s_wt.pol;
        CT = s_wt.pol + ACTOR_TAIL;
    }
    const uint32_t sdelay = clean_env(C, nn) ? 0 : C.sensor_delay;
    const uint32_t cdelay = clean_env(C, nn) ? 0 : C.command_delay;
    // the env's plant for this launch (it changes only at resets, and a
    // reset ends the launch): a row in LDS and its fp64 reciprocals
    constexpr uint32_t PW = sizeof(MdnPhysicsParams) / 4;
    __shared__ float s_ep[DYN ? E : 1][DYN ? PW : 1];
    __shared__ PhysRecip s_erp[DYN ? E : 1];
    if constexpr (DYN) {
        const float* src = reinterpret_cast<const float*>(a.env_phys + nn);
        constexpr uint32_t PR = (PW + G - 1) / G;
        float pv[PR];
#pragma unroll
        for (uint32_t j = 0; j < PR; j++) pv[j] = src[lane + G * j < PW ? lane + G * j : 0];
#pragma unroll
        for (uint32_t j = 0; j < PR; j++)
            if (lane + G * j < PW) s_ep[grp][lane + G * j] = pv[j];
        if (lane == 0) s_erp[grp] = phys_recip(a.env_phys[nn]);
    }
    group_sync();

    // whether some env of the workgroup was reset (or the launch is starting),
    // so that the critic at s must be evaluated this tick
    bool wg_reset = true;
    // fused kernels: the next values of a tick with no reset in the workgroup
    // are formed by the next tick's critic at s (the same critic
    // observations); `deferred` is workgroup-uniform, `prev_due` says that
    // this env's previous row awaits its next value
    bool deferred = false, prev_due = false;
    bool co_fresh = false;  // s_co holds this env's critic observation of its current state
    size_t prev_row = 0;
    for (uint32_t t = 0; t < a.count; t++) {
        const uint32_t tick = SPLIT ? (a.tick0 + t) % a.horizon : t % a.horizon;
        const size_t row = size_t(tick) * N + nn;
        const bool active = live && !(C.eval && r.episodes);
        // depth and observation of this tick still to do
        const bool observe = !SPLIT || t != 0 || !(a.split & SPLIT_BEGIN_AT_ACT);
        const uint32_t count = min(float_bits(world[160]), 16u);  // slots of WWorld

        // this lane's obstacle record (slot `lane` of the world, in range for
        // G <= 16) and whether every env of the wavefront can take the
        // register-held box clearance this tick
        float orec[10];
#pragma unroll
        for (int j = 0; j < 10; j++) orec[j] = world[10 * (lane % 16) + j];
        const bool omine = lane < count;
        const bool fastclr = __all(count <= uint32_t(G) && (!omine || float_bits(orec[0]) == 0u));
        auto clearance = [&](V p, float time) {
            return fastclr ? clearance_boxes<G>(orec, omine, p, time) : clearance_group<G>(world, count, p, time, lane);
        };

        // ---- obstacle centres at the current time (world.hpp:32-41)
        if (active && observe) {
            if (count <= uint32_t(G)) {
                if (omine) {
                    const V c = obstacle_center(world + 10 * lane, r.elapsed);
                    s_cent[grp][3 * lane] = c.x; s_cent[grp][3 * lane + 1] = c.y; s_cent[grp][3 * lane + 2] = c.z;
                }
            } else {
                for (uint32_t i = lane; i < count; i += G) {
                    const V c = obstacle_center(world + 10 * i, r.elapsed);
                    s_cent[grp][3 * i] = c.x; s_cent[grp][3 * i + 1] = c.y; s_cent[grp][3 * i + 2] = c.z;
                }
            }
        }
        group_sync();

        // ---- depth (sim.metal:145-158)
        float R[9];
        rotation(s.q, R);
        const bool depth_now = active && observe && r.steps % C.sensor_period == 0;
        // ray-cast path: when every env of the wavefront casting this tick has
        // a boxes-only world, the wavefront casts its envs' frames one env at a
        // time over all its lanes, each 4-column strip of the frame testing
        // only the boxes that can reach it; else each lane casts the four rays
        // of its pooled 2x2 blocks through the per-kind LDS tables (envs whose
        // world they cannot hold take the generic cast).  The env's
        // observation row is free until observe and holds the tables.
        const bool boxes = boxes_only(world, count);
        const bool wave_boxes = !__any(depth_now && !boxes);
        // else: every casting env's world tabulated for the strip-culled cast
        const bool wave_strips = !wave_boxes && !__any(depth_now && !strip_castable(world, count));
        const float mx = a.mount_x;  // sim.metal:149-152
        const V origin = mk(s.p[0] + mx * R[0], s.p[1] + mx * R[3], s.p[2] + mx * R[6]);
        if (depth_now && lane == 0) {
            float* pose = a.poses + (size_t(nn) * 8 + (r.steps / C.sensor_period) % 8) * 12;
            pose[0] = origin.x; pose[1] = origin.y; pose[2] = origin.z;
#pragma unroll
            for (int j = 0; j < 9; j++) pose[3 + j] = R[j];
        }
        MixCounts mix{0, 0, 0};
        bool mix_ok = false;
        uint32_t NB = 0, NS = 0, NC = 0;
        if (!wave_boxes && !wave_strips) {  // table sizes: the largest counts among the wavefront's casting envs
            if (depth_now) mix_ok = mix_counts(world, count, mix);
            NB = wave_max_u32(mix_ok ? mix.nb : 0u);
            NS = wave_max_u32(mix_ok ? mix.ns : 0u);
            NC = wave_max_u32(mix_ok ? mix.nc : 0u);
        }
        // Wavefront casts (boxes-only or strip tables): lane l takes ray
        // q = l % 4 of block l / 4 of each strip (2 blocks across, 8 down);
        // the env's five depths (one per strip) pass through depth noise and
        // dropout into its sensor ring, and their 2x2 minima into its pooled
        // ring (sim.metal:145-158).
        constexpr uint32_t EW = 64 / G;  // envs per wavefront
        const uint32_t wl = threadIdx.x % 64, wbase = (threadIdx.x / 64) * EW;
        const uint32_t q4 = wl % 4, jb = wl / 4, by = jb / 2, k0 = (2 * by + q4 / 2) * 20 + 2 * (jb % 2) + q4 % 2;
        auto emit_frame = [&](uint32_t ge, uint32_t ne, uint32_t steps_e, uint32_t rng_e, float (&dep)[5]) {
            const uint32_t fidx = steps_e / C.sensor_period;
            const uint32_t slot8 = fidx % 8, slotk = fidx % K;
            const float noise = clean_env(C, ne) ? 0.0f : C.depth_noise;
            const float drop = clean_env(C, ne) ? 0.0f : C.dropout;
            float* ring = a.sensors + (size_t(ne) * 8 + slot8) * PIX;
            if (noise != 0 || drop != 0) {
#pragma unroll
                for (uint32_t st = 0; st < 5; st++) {
                    uint32_t nr = rng_e + (k0 + 4 * st) * 1664525u + steps_e * 1013904223u;
                    dep[st] = clamp_f(dep[st] + noise * normal_draw(nr), 0.0f, 12.0f);
                    if (ur(nr) < drop) dep[st] = 12.0f;
                }
            }
#pragma unroll
            for (uint32_t st = 0; st < 5; st++) {
                const float depth = dep[st];
                ring[k0 + 4 * st] = depth;
                // pooled 2x2 minimum over the quad's lanes (values in [0, 12],
                // never NaN); after the two swaps every lane of the quad holds
                // it, and all four store it (one value to one address)
                float pooled = min_f(depth, bits_float(uint32_t(
                                                __builtin_amdgcn_update_dpp(0, int(float_bits(depth)), 0xB1, 0xF, 0xF, false))));
                pooled = min_f(pooled, bits_float(uint32_t(
                                           __builtin_amdgcn_update_dpp(0, int(float_bits(pooled)), 0x4E, 0xF, 0xF, false))));
                pring(ge)[slotk * POOL + by * 10 + 2 * st + jb % 2] = pooled;
            }
        };
        if (wave_boxes) {
            float* tbl = s_obs[grp];
            uint32_t vis0 = 0, vis1 = 0;  // strip masks, bit 8 st + box (strip 4 in vis1)
            if (depth_now) {
                {   // row 0, the room: the same values in every lane of the group
                    float A[3], B[3];
                    box_slab(world, s_cent[grp], 0, origin, A, B);
#pragma unroll
                    for (int j = 0; j < 3; j++) { tbl[j] = A[j]; tbl[3 + j] = B[j]; }
                }
                // rows 1-8, the boxes: lane l takes box l (rows of absent boxes
                // are written and never read: their strip bits stay 0)
                for (uint32_t i = lane + 1; i < 9; i += G) {
                    float A[3], B[3];
                    box_slab(world, s_cent[grp], i, origin, A, B);
#pragma unroll
                    for (int j = 0; j < 3; j++) { tbl[6 * i + j] = A[j]; tbl[6 * i + 3 + j] = B[j]; }
                    if (i - 1 < count) {
                        const uint32_t m = box_strips(A, B, R, a.tan_v);
                        for (uint32_t st = 0; st < 4; st++) vis0 |= ((m >> st) & 1u) << (8 * st + i - 1);
                        vis1 |= ((m >> 4) & 1u) << (i - 1);
                    }
                }
                vis0 = group_or<G>(vis0);
                vis1 = group_or<G>(vis1);
                // equal values from every lane of the group
                tbl[BOX_TABLE_ORIGIN] = origin.x; tbl[BOX_TABLE_ORIGIN + 1] = origin.y;
                tbl[BOX_TABLE_ORIGIN + 2] = origin.z;
#pragma unroll
                for (int j = 0; j < 9; j++) tbl[BOX_TABLE_ROT + j] = R[j];
                tbl[BOX_TABLE_STRIPS] = bits_float(vis0);
                tbl[BOX_TABLE_STRIPS + 1] = bits_float(vis1);
            }
            const uint64_t casting = __ballot(depth_now);
            group_sync();
            for (uint32_t e = 0; e < EW; e++) {
                if (!((casting >> (e * G)) & 1ull)) continue;
                const uint32_t ge = wbase + e, ne = blockIdx.x * E + ge;
                const float* et = s_obs[ge];
                float SA[9][3], SB[9][3], ER[9];
#pragma unroll
                for (int i = 0; i < 9; i++)
#pragma unroll
                    for (int j = 0; j < 3; j++) { SA[i][j] = et[6 * i + j]; SB[i][j] = et[6 * i + 3 + j]; }
#pragma unroll
                for (int j = 0; j < 9; j++) ER[j] = et[BOX_TABLE_ROT + j];
                const V eo = mk(et[BOX_TABLE_ORIGIN], et[BOX_TABLE_ORIGIN + 1], et[BOX_TABLE_ORIGIN + 2]);
                const uint32_t w0 = __builtin_amdgcn_readfirstlane(float_bits(et[BOX_TABLE_STRIPS]));
                const uint32_t w1 = __builtin_amdgcn_readfirstlane(float_bits(et[BOX_TABLE_STRIPS + 1]));
                const uint32_t steps_e = __builtin_amdgcn_readlane(r.steps, e * G);
                const uint32_t rng_e = __builtin_amdgcn_readlane(r.rng, e * G);
                const uint32_t count_e = __builtin_amdgcn_readfirstlane(min(float_bits(s_world[ge][160]), 16u));
                // the five strips unrolled: no loop branches, and each strip's
                // camera ray is loaded ahead of the strips before it
                float dep[5];
#pragma unroll
                for (uint32_t st = 0; st < 5; st++) {
                    const uint32_t k = k0 + 4 * st;
                    const float rx = CAM[3 * k], ry = CAM[3 * k + 1], rz = CAM[3 * k + 2];
                    const V d = mk(ER[0] * rx + ER[1] * ry + ER[2] * rz, ER[3] * rx + ER[4] * ry + ER[5] * rz,
                                   ER[6] * rx + ER[7] * ry + ER[8] * rz);
                    const bool axes = (__builtin_fabsf(d.x) >= 1e-8f) & (__builtin_fabsf(d.y) >= 1e-8f) &
                                      (__builtin_fabsf(d.z) >= 1e-8f);
                    const uint32_t m = st < 4 ? (w0 >> (8 * st)) & 0xffu : w1 & 0xffu;
                    // one wavefront-uniform branch: every lane's ray takes the
                    // slab path unless some component is below the slab epsilon
                    if (__builtin_expect(__all(axes), 1)) {
                        dep[st] = strip_depth(SA, SB, d, m);
                    } else {
                        // rare: some ray component below the slab epsilon.  The
                        // origin passes through an empty asm so that the generic
                        // cast's per-env set-up stays here instead of being
                        // hoisted into every env's cast
                        V o2 = eo;
                        asm volatile("" : "+v"(o2.x), "+v"(o2.y), "+v"(o2.z));
                        dep[st] = axes ? strip_depth(SA, SB, d, m) : cast_ray(s_world[ge], s_cent[ge], count_e, o2, d);
                    }
                }
                emit_frame(ge, ne, steps_e, rng_e, dep);
            }
        } else if (wave_strips) {
            // any world of at most 16 obstacles: the env's strip table in its
            // observation row (free until observe), lane l taking obstacles
            // l and l + G
            float* tbl = s_obs[grp];
            if (depth_now) {
                uint32_t vm[3] = {0u, 0u, 0u}, kinds = 0u;
                {   // the room: the same values in every lane of the group
                    float A[3], B[3];
                    box_slab(world, s_cent[grp], 0, origin, A, B);
#pragma unroll
                    for (int j = 0; j < 3; j++) { tbl[j] = A[j]; tbl[3 + j] = B[j]; }
                }
                for (uint32_t i = lane; i < count; i += G) {
                    float A[3], B[3];
                    kinds |= strip_entry(world, s_cent[grp], i, origin, tbl + 6 + 6 * i, A, B) << (2 * i);
                    const uint32_t m = box_strips(A, B, R, a.tan_v);
#pragma unroll
                    for (uint32_t st = 0; st < 5; st++) vm[st / 2] |= ((m >> st) & 1u) << (16 * (st % 2) + i);
                }
#pragma unroll
                for (int j = 0; j < 3; j++) vm[j] = group_or<G>(vm[j]);
                kinds = group_or<G>(kinds);
                // equal values from every lane of the group
                tbl[STRIP_TABLE_ORIGIN] = origin.x; tbl[STRIP_TABLE_ORIGIN + 1] = origin.y;
                tbl[STRIP_TABLE_ORIGIN + 2] = origin.z;
#pragma unroll
                for (int j = 0; j < 9; j++) tbl[STRIP_TABLE_ROT + j] = R[j];
#pragma unroll
                for (int j = 0; j < 3; j++) tbl[STRIP_TABLE_MASKS + j] = bits_float(vm[j]);
                tbl[STRIP_TABLE_KINDS] = bits_float(kinds);
            }
            const uint64_t casting = __ballot(depth_now);
            group_sync();
            for (uint32_t e = 0; e < EW; e++) {
                if (!((casting >> (e * G)) & 1ull)) continue;
                const uint32_t ge = wbase + e, ne = blockIdx.x * E + ge;
                const float* et = s_obs[ge];
                float ER[9], RA[3], RB[3];
#pragma unroll
                for (int j = 0; j < 3; j++) { RA[j] = et[j]; RB[j] = et[3 + j]; }
#pragma unroll
                for (int j = 0; j < 9; j++) ER[j] = et[STRIP_TABLE_ROT + j];
                const V eo = mk(et[STRIP_TABLE_ORIGIN], et[STRIP_TABLE_ORIGIN + 1], et[STRIP_TABLE_ORIGIN + 2]);
                uint32_t wm[3];
#pragma unroll
                for (int j = 0; j < 3; j++) wm[j] = __builtin_amdgcn_readfirstlane(float_bits(et[STRIP_TABLE_MASKS + j]));
                const uint32_t kinds_e = __builtin_amdgcn_readfirstlane(float_bits(et[STRIP_TABLE_KINDS]));
                const uint32_t steps_e = __builtin_amdgcn_readlane(r.steps, e * G);
                const uint32_t rng_e = __builtin_amdgcn_readlane(r.rng, e * G);
                const uint32_t count_e = __builtin_amdgcn_readfirstlane(min(float_bits(s_world[ge][160]), 16u));
                float dep[5];
#pragma unroll
                for (uint32_t st = 0; st < 5; st++) {
                    const uint32_t k = k0 + 4 * st;
                    const float rx = CAM[3 * k], ry = CAM[3 * k + 1], rz = CAM[3 * k + 2];
                    const V d = mk(ER[0] * rx + ER[1] * ry + ER[2] * rz, ER[3] * rx + ER[4] * ry + ER[5] * rz,
                                   ER[6] * rx + ER[7] * ry + ER[8] * rz);
                    const bool axes = (__builtin_fabsf(d.x) >= 1e-8f) & (__builtin_fabsf(d.y) >= 1e-8f) &
                                      (__builtin_fabsf(d.z) >= 1e-8f);
                    const uint32_t m = (wm[st / 2] >> (16 * (st % 2))) & 0xffffu;
                    if (__builtin_expect(__all(axes), 1)) {
                        dep[st] = strip_depth_mixed(et, d, m, kinds_e, RA, RB);
                    } else {  // rare: some ray component below the slab epsilon
                        V o2 = eo;
                        asm volatile("" : "+v"(o2.x), "+v"(o2.y), "+v"(o2.z));
                        dep[st] = axes ? strip_depth_mixed(et, d, m, kinds_e, RA, RB)
                                       : cast_ray(s_world[ge], s_cent[ge], count_e, o2, d);
                    }
                }
                emit_frame(ge, ne, steps_e, rng_e, dep);
            }
        } else if (depth_now) {
            const uint32_t fidx = r.steps / C.sensor_period;
            const uint32_t slot8 = fidx % 8, slotk = fidx % K;
            const float noise = clean_env(C, nn) ? 0.0f : C.depth_noise;
            const float drop = clean_env(C, nn) ? 0.0f : C.dropout;
            float* ring = a.sensors + (size_t(nn) * 8 + slot8) * PIX;
            float* tbl = s_obs[grp];
            float RA[3], RB[3];
            if (mix_ok) {
                mix_table(world, s_cent[grp], count, origin, NB, NS, lane, G, tbl);
                const float pr[3] = {origin.x - 6.0f, origin.y - 0.0f, origin.z - 2.5f}, er[3] = {8.0f, 5.0f, 2.5f};
#pragma unroll
                for (int j = 0; j < 3; j++) { RA[j] = -er[j] - pr[j]; RB[j] = er[j] - pr[j]; }
            }
            group_sync();
            for (uint32_t b = lane; b < POOL; b += G) {
                const uint32_t y = (b / 10) * 2, x = (b % 10) * 2;
                float pooled = 12.0f;
                // the block's four rays through the per-kind tables together
                float mixed[4] = {0, 0, 0, 0};
                bool block_mixed = false;
                if (mix_ok) {
                    V dq[4];
                    bool all_axes = true;
#pragma unroll
                    for (uint32_t q4 = 0; q4 < 4; q4++) {
                        const uint32_t k = (y + q4 / 2) * 20 + x + q4 % 2;
                        const float rx = CAM[3 * k], ry = CAM[3 * k + 1], rz = CAM[3 * k + 2];
                        dq[q4] = mk(R[0] * rx + R[1] * ry + R[2] * rz, R[3] * rx + R[4] * ry + R[5] * rz,
                                    R[6] * rx + R[7] * ry + R[8] * rz);
                        all_axes = all_axes && (__builtin_fabsf(dq[q4].x) >= 1e-8f) &&
                                   (__builtin_fabsf(dq[q4].y) >= 1e-8f) && (__builtin_fabsf(dq[q4].z) >= 1e-8f);
                    }
                    block_mixed = all_axes;
                    if (block_mixed) cast_block_mixed(RA, RB, tbl, mix, NB, NS, NC, dq, mixed);
                }
#pragma unroll
                for (uint32_t dy = 0; dy < 2; dy++)
#pragma unroll
                    for (uint32_t dx = 0; dx < 2; dx++) {
                        const uint32_t k = (y + dy) * 20 + x + dx;
                        const float rx = CAM[3 * k], ry = CAM[3 * k + 1], rz = CAM[3 * k + 2];
                        const V d = mk(R[0] * rx + R[1] * ry + R[2] * rz, R[3] * rx + R[4] * ry + R[5] * rz,
                                       R[6] * rx + R[7] * ry + R[8] * rz);
                        float depth;
                        const bool axes = (__builtin_fabsf(d.x) >= 1e-8f) & (__builtin_fabsf(d.y) >= 1e-8f) &
                                          (__builtin_fabsf(d.z) >= 1e-8f);
                        if (block_mixed)
                            depth = mixed[dy * 2 + dx];
                        else if (mix_ok && axes)
                            depth = cast_ray_mixed(RA, RB, tbl, mix, NB, NS, NC, d);
                        else
                            depth = cast_ray(world, s_cent[grp], count, origin, d);
                        if (noise != 0 || drop != 0) {
                            uint32_t nr = r.rng + k * 1664525u + r.steps * 1013904223u;
                            depth = clamp_f(depth + noise * normal_draw(nr), 0.0f, 12.0f);
                            if (ur(nr) < drop) depth = 12.0f;
                        }
                        ring[k] = depth;
                        pooled = min_f(pooled, depth);
                    }
                pring(grp)[slotk * POOL + b] = pooled;
            }
        }
        group_sync();

        // ---- observe (sim.metal:182-228, pooled actor inputs + optional hint)
        const uint32_t available = r.steps / C.sensor_period;
        const uint32_t frame = available > sdelay ? available - sdelay : 0;
        const uint32_t prev = frame > 0 ? frame - 1 : 0;
        const bool have = available >= sdelay;
        float* og = a.obs + row * D;
        if (active && observe) {
            static_assert(POOL % G == 0, "whole pooled rows per lane");
#pragma unroll
            for (uint32_t bi = 0; bi < POOL / G; bi++) {
                const uint32_t b = lane + G * bi;
                const float* rg = pring(grp);
                const float cur = have ? div_r(rg[(frame % K) * POOL + b], 1.0 / 12.0) : 1.0f;
                // mode 18 (sim.metal:211-213): evaluation without the previous frame
                const float pre = C.mode == 18 ? cur : have ? div_r(rg[(prev % K) * POOL + b], 1.0 / 12.0) : 1.0f;
                s_obs[grp][b] = cur;
                s_obs[grp][POOL + b] = pre;
                og[b] = cur;
                og[POOL + b] = pre;
            }
            const float* gw = world + 163;
            const float dx = gw[0] - s.p[0], dy = gw[1] - s.p[1], dz = gw[2] - s.p[2];
            const float distance = max_f(sqrt_f(dx * dx + dy * dy + dz * dz), 1.0e-6f);
            float ctx[21];
#pragma unroll
            for (int j = 0; j < 3; j++) {
                ctx[j] = (R[j] * dx + R[3 + j] * dy + R[6 + j] * dz) / distance;
                ctx[4 + j] = (R[j] * s.v[0] + R[3 + j] * s.v[1] + R[6 + j] * s.v[2]) / 4.0f;
                ctx[7 + j] = s.w[j] / 4.0f;
                ctx[10 + j] = R[6 + j];
            }
            ctx[3] = min_f(div_r(distance, 1.0 / 10.0), 1.5f);
#pragma unroll
            for (int j = 0; j < 4; j++) ctx[13 + j] = r.prev_nav[j];
            ctx[17] = float(r.steps - frame * C.sensor_period) * P.dt * float(C.substeps);
            const float ref0 = r.ref_pos[0] - s.p[0], ref1 = r.ref_pos[1] - s.p[1], ref2 = r.ref_pos[2] - s.p[2];
#pragma unroll
            for (int j = 0; j < 3; j++) ctx[18 + j] = __builtin_amdgcn_fmed3f((R[j] * ref0 + R[3 + j] * ref1 + R[6 + j] * ref2) * 2.0f, -1.0f, 1.0f);
#pragma unroll
            // every lane of the group holds the same values and writes them
            // (equal stores to one address; cheaper than per-value owner branches)
            for (int j = 0; j < 21; j++) { s_obs[grp][2 * POOL + j] = ctx[j]; og[2 * POOL + j] = ctx[j]; }
            if (D == MDN_ACTOR_OBS_PRIOR && a.mem_head) {  // geometry-memory hint: computed outside
                uint32_t* hd = a.mem_head + size_t(nn) * MEM_HEAD_WORDS;
                uint32_t valid = have ? min(frame + 1, 8u - sdelay) : 0u;
                if (C.mode == 18) valid = min(valid, 1u);  // memory.metal:34: newest frame only
                if (lane == 0) {
                    hd[MEM_HEAD_OBSERVED] = 1u;
                    hd[MEM_HEAD_FRAME] = frame;
                    hd[MEM_HEAD_VALID] = valid;
                    hd[MEM_HEAD_DISTANCE] = float_bits(distance);
#pragma unroll
                    for (int j = 0; j < 3; j++) hd[MEM_HEAD_POSE + j] = float_bits(s.p[j]);
#pragma unroll
                    for (int j = 0; j < 9; j++) hd[MEM_HEAD_POSE + 3 + j] = float_bits(R[j]);
                }
            } else if constexpr (D == MDN_ACTOR_OBS_PRIOR) {  // geometry-prior hint (sim.metal:226)
                group_sync();                          // the group's pooled ranges are in s_obs
                const float goal3[3] = {ctx[0], ctx[1], ctx[2]};
                const float vel3[3] = {ctx[4] * 4.0f, ctx[5] * 4.0f, ctx[6] * 4.0f};
                float hint[3];
                guidance_group<G>(s_obs[grp], a.cells, goal3, distance, vel3, a.sensor_dt, a.inv_sensor_dt, lane, hint);
#pragma unroll
                for (int j = 0; j < 3; j++) { s_obs[grp][D - 3 + j] = hint[j]; og[D - 3 + j] = hint[j]; }
            }
            // critic observation (sim.metal:159-181).  When the previous tick
            // of this launch formed it as its next state's and did not reset
            // the env, s_co already holds it (the same operations on the same
            // state, time and step count) and it is only stored.
            float* cg = a.co + row * COBS;
            if (co_fresh) {
#pragma unroll
                for (int j = 0; j < 32; j++) cg[j] = s_co[grp][j];
            } else {
                float cob[COBS];
#pragma unroll
                for (int j = 0; j < 32; j++) cob[j] = 0;
#pragma unroll
                for (int j = 0; j < 3; j++) {
                    cob[j] = div_r(gw[j] - s.p[j], 1.0 / 10.0);
                    cob[j + 3] = s.v[j] / 4.0f;
                    cob[j + 6] = s.w[j] / 4.0f;
                    cob[j + 13] = div_r(s.p[j], 1.0 / 10.0);
                    cob[j + 16] = (r.ref_pos[j] - s.p[j]) * 2.0f;
                }
#pragma unroll
                for (int j = 0; j < 4; j++) cob[9 + j] = s.q[j];
                cob[30] = world[166];
                cob[31] = world[167];
                cob[19] = div_r(clearance(mk(s.p[0], s.p[1], s.p[2]), r.elapsed), 1.0 / 5.0);
                cob[20] = div_r(float(r.steps), 1.0 / 200.0);
#pragma unroll
                for (uint32_t j = 0; j < 3; j++)
                    if (j < count) {
                        cob[21 + j * 3] = div_r(s_cent[grp][3 * j] - s.p[0], 1.0 / 10.0);
                        cob[22 + j * 3] = div_r(s_cent[grp][3 * j + 1] - s.p[1], 1.0 / 10.0);
                        cob[23 + j * 3] = div_r(s_cent[grp][3 * j + 2] - s.p[2], 1.0 / 10.0);
                    }
#pragma unroll
                for (int j = 0; j < 32; j++) { s_co[grp][j] = cob[j]; cg[j] = cob[j]; }
            }
        } else if (SPLIT && active) {  // begins at act: this tick's rows as written before
            // (fixed trip counts, every load issued before the first store)
            constexpr uint32_t OR = (D + G - 1) / G, CR = (COBS + G - 1) / G;
            float ov[OR], cv[CR];
#pragma unroll
            for (uint32_t j = 0; j < OR; j++) ov[j] = og[lane + G * j < D ? lane + G * j : 0];
#pragma unroll
            for (uint32_t j = 0; j < CR; j++) cv[j] = a.co[row * COBS + (lane + G * j < COBS ? lane + G * j : 0)];
#pragma unroll
            for (uint32_t j = 0; j < OR; j++)
                if (lane + G * j < D) s_obs[grp][lane + G * j] = ov[j];
#pragma unroll
            for (uint32_t j = 0; j < CR; j++)
                if (lane + G * j < COBS) s_co[grp][lane + G * j] = cv[j];
        } else if (D == MDN_ACTOR_OBS_PRIOR && live && observe && a.mem_head && lane == 0) {
            a.mem_head[size_t(nn) * MEM_HEAD_WORDS + MEM_HEAD_OBSERVED] = 0u;
        }
        group_sync();
        if (SPLIT && t + 1 == a.count && (a.split & SPLIT_END_AFTER_OBSERVE)) break;

        // ---- actor and critic hidden layers (ppo.hpp:65-72, 82-89)
        if constexpr (X) {
            // means come from the caller's policy
        } else if constexpr (W > 1) {  // all 32 envs of the workgroup on the matrix cores
            static_assert(E == 32, "matrix-core layers assume 32 envs per workgroup");
            __syncthreads();
            wg_layer<D, OS, HID + 1>(&s_obs[0][0], AW1, AT, &s_ah[0][0]);
            // When no env of the workgroup was reset at the end of the previous
            // tick of this launch, every env's critic observation now is the
            // one that tick evaluated as its next state (the same operations on
            // the same state, time and step count), so the values it left in
            // s_x[env][4] are this tick's values; else evaluate the critic.
            // After a tick whose next values were deferred, the critic at s
            // forms them too: an env active now has the same critic
            // observation, an env that went inactive kept its row.
            const bool critic_s = wg_reset || deferred;
            if (critic_s) wg_layer_rb<COBS, COBS + 1, HID + 1>(&s_co[0][0], cw1, CT, &s_ch[0][0]);
            __syncthreads();
            // heads: means (waves 0-1) and value (waves 2-3) into s_x[env][0..4]
            wg_head<4, HID + 1>(&s_ah[0][0], AT + HID, HID, AT + 5 * HID, 0, &s_x[0][0], 0);
            if (critic_s) wg_head<1, HID + 1>(&s_ch[0][0], CT + HID, 0, CT + 2 * HID, 2, &s_x[0][0], 4);
            __syncthreads();
            if (deferred && prev_due && lane == 0) a.next_values[prev_row] = s_x[grp][4];
        } else if (active) {
            float acc[HU];
#pragma unroll
            for (int k = 0; k < HU; k++) acc[k] = A[a_b1 + lane * HU + k];
#pragma unroll 4
            for (uint32_t i = 0; i < D; i++) {
                const float x = s_obs[grp][i];
                const float* w = AW1 + i * HID + lane * HU;
#pragma unroll
                for (int k = 0; k < HU; k++) acc[k] = fma_f(w[k], x, acc[k]);
            }
#pragma unroll
            for (int k = 0; k < HU; k++) s_ah[grp][lane * HU + k] = tanh_f(acc[k]);
#pragma unroll
            for (int k = 0; k < HU; k++) acc[k] = CR[c_b1 + lane * HU + k];
#pragma unroll 4
            for (uint32_t i = 0; i < COBS; i++) {
                const float x = s_co[grp][i];
                const float* w = a.critic_w1t + size_t(i) * HID + lane * HU;
#pragma unroll
                for (int k = 0; k < HU; k++) acc[k] = fma_f(w[k], x, acc[k]);
            }
#pragma unroll
            for (int k = 0; k < HU; k++) s_ch[grp][lane * HU + k] = tanh_f(acc[k]);
        }
        group_sync();

        // ---- act (sim.metal:229-256): means, value, sample, log-prob, command
        float a_cmd[4] = {0, 0, 0, 0};
        if (active) {
            float mean[4], value = 0.0f;
            if constexpr (X) {
#pragma unroll
                for (int q = 0; q < 4; q++) mean[q] = a.ext_means[row * 4 + q];
            } else if constexpr (W > 1) {
#pragma unroll
                for (int q = 0; q < 4; q++) mean[q] = s_x[grp][q];
                if constexpr (D == MDN_ACTOR_OBS_PRIOR)  // ppo.hpp:77
#pragma unroll
                    for (int q = 0; q < 3; q++) mean[q] += s_obs[grp][D - 3 + q];
                value = s_x[grp][4];
            } else {
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    float z = A[a_b2 + q];
#pragma unroll 8
                    for (uint32_t h = 0; h < HID; h++) z = fma_f(A[a_w2 + q * HID + h], s_ah[grp][h], z);
                    if (D == MDN_ACTOR_OBS_PRIOR && q < 3) z += s_obs[grp][D - 3 + q];  // ppo.hpp:77
                    mean[q] = z;
                }
                value = CR[c_b2];
#pragma unroll 8
                for (uint32_t h = 0; h < HID; h++) value = fma_f(CR[c_w2 + h], s_ch[grp][h], value);
            }
            float deployed = 1.0f;
            if constexpr (D == MDN_ACTOR_OBS_PRIOR) {
                if (C.mode >= 9 && C.mode <= 21) guided_mode_means(C.mode, s_obs[grp], mean);
                // sim.metal:234-238, 246-252: mode 22 trains through the
                // deployed mode-17 map of the sample (log-probability of the raw one)
                if (C.mode == 22) deployed = 0.25f + 0.75f * (overhead_cells(s_obs[grp]) / 20.0f);
            }
            // The four actions are drawn in parallel: lane j of each quad
            // takes action j from the stream state the sequential draw would
            // have reached (each action draws one normal, two xorshift steps,
            // in the sampling modes), and the quad exchanges the results.
            const bool draws = C.mode == 0 || C.mode == 22 || C.mode == 1;
            uint32_t rs[5];
            rs[0] = r.rng;
#pragma unroll
            for (int q = 1; q < 5; q++) {
                uint32_t x = rs[q - 1];
                xs(x);
                xs(x);
                rs[q] = draws ? x : rs[q - 1];
            }
            static_assert(G % 4 == 0, "whole quads per lane group");
            const uint32_t jl = lane % 4;
            uint32_t rng = jl == 0 ? rs[0] : jl == 1 ? rs[1] : jl == 2 ? rs[2] : rs[3];
            const float mj = jl == 0 ? mean[0] : jl == 1 ? mean[1] : jl == 2 ? mean[2] : mean[3];
            const float ls = X ? a.ext_log_std[jl] : AT[5 * HID + 4 + jl];
            float sd, isd;
            if constexpr (W > 1 && !X) {
                sd = s_wt.pol[ACTOR_TAIL + CRITIC_TAIL + jl];
                isd = s_wt.pol[ACTOR_TAIL + CRITIC_TAIL + 4 + jl];
            } else {
                sd = exp_f(ls);
                isd = exp_f(-ls);
            }
            float actj = mj + ((C.mode == 0 || C.mode == 22) ? sd * normal_draw(rng) : 0.0f);
            if (C.mode == 1) actj = normal_draw(rng);
            const float diff = (actj - mj) * isd;
            const float term = -0.5f * (diff * diff + 2 * ls + LOG_TWO_PI);
            float executed = actj;
            if (D == MDN_ACTOR_OBS_PRIOR && C.mode == 22) {
                const float prior = s_obs[grp][D - 3 + (jl < 3 ? jl : 0)];
                executed = jl < 3 ? prior + deployed * (actj - prior) : deployed * actj;
            }
            const float cmdj = tanh_f(executed);
            // quad broadcasts (DPP quad_perm [q,q,q,q]); log-probability terms
            // summed in action order, as the sequential loop does
            float lp = 0;
            const float act[4] = {quad_bcast<0>(actj), quad_bcast<1>(actj), quad_bcast<2>(actj), quad_bcast<3>(actj)};
            a_cmd[0] = quad_bcast<0>(cmdj); a_cmd[1] = quad_bcast<1>(cmdj);
            a_cmd[2] = quad_bcast<2>(cmdj); a_cmd[3] = quad_bcast<3>(cmdj);
            lp += quad_bcast<0>(term);
            lp += quad_bcast<1>(term);
            lp += quad_bcast<2>(term);
            lp += quad_bcast<3>(term);
            r.rng = rs[4];
            if (C.mode == 2 || C.mode == 3 || C.mode == 20) {  // sim.metal:257-262
                float dd[3] = {world[163] - s.p[0], world[164] - s.p[1], world[165] - s.p[2]};
                const float ln = sqrt_f(dd[0] * dd[0] + dd[1] * dd[1] + dd[2] * dd[2]);
                const float inv = 1.0f / ln, lim = min_f(ln, C.speed);
#pragma unroll
                for (int j = 0; j < 3; j++) dd[j] = (dd[j] * inv) * lim;
                a_cmd[0] = (R[0] * dd[0] + R[3] * dd[1] + R[6] * dd[2]) / C.speed;
                a_cmd[1] = (R[1] * dd[0] + R[4] * dd[1] + R[7] * dd[2]) / C.speed;
                a_cmd[2] = (R[2] * dd[0] + R[5] * dd[1] + R[8] * dd[2]) / C.speed;
                a_cmd[3] = 0;
            }
            if (lane == 0) {
#pragma unroll
                for (int j = 0; j < 4; j++) a.actions[row * 4 + j] = act[j];
                a.logp[row] = lp;
                if constexpr (!X) a.values[row] = value;
                const uint32_t slot = r.steps % 8;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    s_cmd[grp][slot * 4 + j] = a_cmd[j];
                    a.commands[size_t(nn) * 32 + slot * 4 + j] = a_cmd[j];
                }
            }
        }
        group_sync();
        if (active) {  // sim.metal:263-270
            const uint32_t applied = r.steps > cdelay ? r.steps - cdelay : 0;
#pragma unroll
            for (int j = 0; j < 4; j++) r.prev_nav[j] = r.steps < cdelay ? 0.0f : s_cmd[grp][(applied % 8) * 4 + j];
            float v[3] = {r.prev_nav[0] * C.speed, r.prev_nav[1] * C.speed,
                          r.prev_nav[2] * C.speed * (C.velocity_contract == 0 ? 0.5f : 1.0f)};
            if (C.velocity_contract == 1) {
                const float m = sqrt_f(v[0] * v[0] + v[1] * v[1] + v[2] * v[2]);
                const float scale = min_f(1.0f, C.speed / max_f(m, 1e-8f));
#pragma unroll
                for (int j = 0; j < 3; j++) v[j] *= scale;
            }
            if (C.mode == 19) {
                const float m = sqrt_f(v[0] * v[0] + v[1] * v[1] + v[2] * v[2]);
                if (m > 1e-8f) {
                    const float scale = C.speed / m;
#pragma unroll
                    for (int j = 0; j < 3; j++) v[j] *= scale;
                }
            }
#pragma unroll
            for (int j = 0; j < 3; j++) r.desired_vel[j] = R[j * 3] * v[0] + R[j * 3 + 1] * v[1] + R[j * 3 + 2] * v[2];
            r.yaw += r.prev_nav[3] * P.dt * float(C.substeps) * 0.5f;
        }

        // ---- advance (sim.metal:272-304): substeps of RAPTOR + RK4
        const float gx = world[163], gy = world[164], gz = world[165];
        float before = 0;
        {
            const float dx = gx - s.p[0], dy = gy - s.p[1], dz = gz - s.p[2];
            before = sqrt_f(dx * dx + dy * dy + dz * dz);
        }
        float si, c, sh, ch;
        sincos_f(r.yaw, &si, &c);
        sincos_f(r.yaw * 0.5f, &sh, &ch);
        bool collision = false, done = !active;
        float step_clearance = 12.0f;
        const MdnPhysicsParams& EP = DYN ? *reinterpret_cast<const MdnPhysicsParams*>(&s_ep[grp][0]) : P;
        const float wind[3] = {world[166] * EP.mass, world[167] * EP.mass, world[168] * EP.mass};
        // the standard-structure derivative takes wind / mass, the same
        // division physics.hpp:101 repeats in every derivative evaluation
        const float wm[3] = {div_r(wind[0], RP.mass), div_r(wind[1], RP.mass), div_r(wind[2], RP.mass)};
        bool nzero = no_negative_zero(s);  // no component of s is -0 (derivative_quad's condition)
        for (uint32_t step = 0; step < C.substeps; step++) {
            float mo[22] = {0};
            if (!done) {
                const float v0 = r.desired_vel[0], v1 = r.desired_vel[1], v2 = r.desired_vel[2];
                r.ref_pos[0] += v0 * P.dt; r.ref_pos[1] += v1 * P.dt; r.ref_pos[2] += v2 * P.dt;
                const float dp0 = s.p[0] - r.ref_pos[0], dp1 = s.p[1] - r.ref_pos[1], dp2 = s.p[2] - r.ref_pos[2];
                const float dv0 = s.v[0] - v0, dv1 = s.v[1] - v1, dv2 = s.v[2] - v2;
                // clamps to nonzero bounds of finite values: the median of three
                mo[0] = __builtin_amdgcn_fmed3f(c * dp0 + si * dp1, -.5f, .5f);
                mo[1] = __builtin_amdgcn_fmed3f(-si * dp0 + c * dp1, -.5f, .5f);
                mo[2] = __builtin_amdgcn_fmed3f(dp2, -.5f, .5f);
                const float q[4] = {ch * s.q[0] + sh * s.q[3], ch * s.q[1] + sh * s.q[2], ch * s.q[2] - sh * s.q[1],
                                    ch * s.q[3] - sh * s.q[0]};
                rotation(q, mo + 3);
                mo[12] = __builtin_amdgcn_fmed3f(c * dv0 + si * dv1, -1.0f, 1.0f);
                mo[13] = __builtin_amdgcn_fmed3f(-si * dv0 + c * dv1, -1.0f, 1.0f);
                mo[14] = __builtin_amdgcn_fmed3f(dv2, -1.0f, 1.0f);
                mo[15] = s.w[0]; mo[16] = s.w[1]; mo[17] = s.w[2];
#pragma unroll
                for (int j = 0; j < 4; j++) mo[18 + j] = r.motors[j];
            }
            float act[4];
            if constexpr (W > 1)
                raptor_wave<G, OS>(RW, rops, mo, &s_obs[0][0], &s_x[0][0], &s_rh[0][0], grp, lane, !done, act);
            else
                raptor_group<G>(RW, mo, r.hidden, hu, s_x[grp], s_h[grp], lane, !done, act);
            if (!done) {
#pragma unroll
                for (int q = 0; q < 4; q++) r.motors[q] = act[q];
                State nx;
                if constexpr (DYN) physics_step(EP, s_erp[grp], s, act, wind, nx);
                else if ((CF || a.quad) && !__any(!nzero)) physics_step<true>(P, RP, s, act, wm, nx);
                else physics_step(P, RP, s, act, wind, nx);
                // every component finite (isfinite_f) and none -0, in integer
                // form: the largest exponent field and the smallest bits ^ sign
                const float* nf = &nx.p[0];
                uint32_t emax = 0u, zmin = 0xffffffffu;
#pragma unroll
                for (int j = 0; j < 17; j++) {
                    const uint32_t u = float_bits(nf[j]);
                    emax = max(emax, u & 0x7f800000u);
                    zmin = min(zmin, u ^ 0x80000000u);
                }
                const bool valid = emax != 0x7f800000u;
                if (!valid) {
                    collision = true;
                    done = true;
                } else {
                    const float ex = s.p[0] - nx.p[0], ey = s.p[1] - nx.p[1], ez = s.p[2] - nx.p[2];
                    r.path += sqrt_f(ex * ex + ey * ey + ez * ez);
                    s = nx;
                    nzero = zmin != 0u;
                    r.elapsed += P.dt;
                    const float cl = clearance(mk(s.p[0], s.p[1], s.p[2]), r.elapsed);
                    step_clearance = min_f(step_clearance, cl);
                    r.min_clearance = min_f(r.min_clearance, cl);
                    r.peak_speed = max_f(r.peak_speed, sqrt_f(s.v[0] * s.v[0] + s.v[1] * s.v[1] + s.v[2] * s.v[2]));
                    if (cl <= 0) {
                        collision = true;
                        done = true;
                    }
                }
            }
        }

        // ---- outcome (sim.metal:304-306), next value, episode end
        bool ended = false;
        if (active) {
            r.steps++;
            const float dx = gx - s.p[0], dy = gy - s.p[1], dz = gz - s.p[2];
            const float after = sqrt_f(dx * dx + dy * dy + dz * dz);
            bool success = after < (C.mode == 20 ? .10f : .35f) && !collision;
            bool timeout = r.steps >= C.max_steps;
            float reward = (before - after) * 2.0f - .01f -
                           C.risk_coef * clamp_f((0.6f - step_clearance) / 0.6f, 0.0f, 1.0f) +
                           (success ? 10.0f : 0.0f) - (collision ? 10.0f : 0.0f);
            if constexpr (DYN) {
                if (a.task_cfg) {  // sim.metal:307-315
                    const float executed[4] = {r.desired_vel[0], r.desired_vel[1], r.desired_vel[2], r.prev_nav[3] * 0.5f};
                    const TaskOutcome o = task_step(a.task_states + nn, *a.task_cfg, s.p, s.v, executed, collision,
                                                    timeout, lane == 0);
                    success = o.stable_success && !collision;
                    timeout = o.timeout;
                    reward = o.reward;
                }
            }
            const bool term = collision || success;
            const bool trunc = timeout && !term;
            if (lane == 0) {
                a.rewards[row] = reward;
                a.terminated[row] = term ? 1 : 0;
                a.truncated[row] = trunc ? 1 : 0;
                if constexpr (DYN)  // sim.metal:317
                    a.bank_transition[row] = a.bank_active ? a.bank_active[nn] : MDN_BANK_REHEARSAL;
            }
            // critic observation of the next state (time elapsed after the substeps)
            float cob[COBS];
#pragma unroll
            for (int j = 0; j < 32; j++) cob[j] = 0;
#pragma unroll
            for (int j = 0; j < 3; j++) {
                cob[j] = div_r(world[163 + j] - s.p[j], 1.0 / 10.0);
                cob[j + 3] = s.v[j] / 4.0f;
                cob[j + 6] = s.w[j] / 4.0f;
                cob[j + 13] = div_r(s.p[j], 1.0 / 10.0);
                cob[j + 16] = (r.ref_pos[j] - s.p[j]) * 2.0f;
            }
#pragma unroll
            for (int j = 0; j < 4; j++) cob[9 + j] = s.q[j];
            cob[30] = world[166];
            cob[31] = world[167];
            cob[19] = div_r(clearance(mk(s.p[0], s.p[1], s.p[2]), r.elapsed), 1.0 / 5.0);
            cob[20] = div_r(float(r.steps), 1.0 / 200.0);
#pragma unroll
            for (uint32_t j = 0; j < 3; j++)
                if (j < count) {
                    const V cc = obstacle_center(world + 10 * j, r.elapsed);
                    cob[21 + j * 3] = div_r(cc.x - s.p[0], 1.0 / 10.0);
                    cob[22 + j * 3] = div_r(cc.y - s.p[1], 1.0 / 10.0);
                    cob[23 + j * 3] = div_r(cc.z - s.p[2], 1.0 / 10.0);
                }
            float* ncg = a.nco + row * COBS;
#pragma unroll
            for (int j = 0; j < 32; j++) { s_co[grp][j] = cob[j]; ncg[j] = cob[j]; }
            if (success || collision || timeout) {  // sim.metal:328-331
                r.successes += success;
                r.collisions += collision;
                r.timeouts += trunc;
                r.episodes++;
                r.success_time += success ? r.elapsed : 0;
                r.total_path += r.path;
                r.total_elapsed += r.elapsed;
                r.final_progress += 1.0f - after / max_f(r.initial_distance, 1.0e-4f);
                ended = !C.eval;
            }
        }
        co_fresh = active && !ended;
        if constexpr (X) {
            // next values are the caller's (from the stored next critic observations)
        } else if constexpr (W > 1) {  // next value: critic hidden of s' for all 32 envs
            wg_reset = __syncthreads_or(ended) != 0;
            // with no reset in the workgroup and another tick to come in this
            // launch, the next tick's critic at s forms these next values
            // (a launch without split-tick flags observes every tick and runs
            // to its last tick, so the guided actor's fused launches qualify)
            deferred = (!SPLIT || a.split == 0u) && !wg_reset && t + 1 < a.count;
            if (!deferred) {
                wg_layer_rb<COBS, COBS + 1, HID + 1>(&s_co[0][0], cw1, CT, &s_ch[0][0]);
                __syncthreads();
                wg_head<1, HID + 1>(&s_ch[0][0], CT + HID, 0, CT + 2 * HID, 0, &s_x[0][0], 4);
                __syncthreads();
            }
        } else {  // next value: critic hidden split over the group
            group_sync();
            if (active) {
                float acc[HU];
#pragma unroll
                for (int k = 0; k < HU; k++) acc[k] = CR[c_b1 + lane * HU + k];
#pragma unroll 4
                for (uint32_t i = 0; i < COBS; i++) {
                    const float x = s_co[grp][i];
                    const float* w = a.critic_w1t + size_t(i) * HID + lane * HU;
#pragma unroll
                    for (int k = 0; k < HU; k++) acc[k] = fma_f(w[k], x, acc[k]);
                }
#pragma unroll
                for (int k = 0; k < HU; k++) s_ch[grp][lane * HU + k] = tanh_f(acc[k]);
            }
            group_sync();
        }
        uint32_t reset_rng = 0, reset_family = 0, reset_seed = 0;
        prev_due = deferred && active;
        prev_row = row;
        if (active) {
            if constexpr (!X) {
                float value;
                if constexpr (W > 1) {
                    value = s_x[grp][4];
                } else {
                    value = CR[c_b2];
#pragma unroll 8
                    for (uint32_t h = 0; h < HID; h++) value = fma_f(CR[c_w2 + h], s_ch[grp][h], value);
                }
                if (!deferred && lane == 0) a.next_values[row] = value;
            }
            if (ended) {
                reset_rng = r.rng;
                reset_draw(C, nn, false, reset_rng, reset_family, reset_seed);
                if (lane == 0) {
                    WorldGen wg{world};
                    wg.generate(reset_seed, reset_family, C.distance);
                }
            }
        }
        group_sync();
        if (ended) {  // sim_reset_one, not first
            reset_apply(C, P, RW, nn, false, reset_rng, world, s, r);
#pragma unroll
            for (int j = 0; j < U; j++) hu[j] = RW[2000 + lane + G * j];
            if constexpr (W > 1)
                for (uint32_t c = lane; c < 16; c += G) s_rh[grp][c] = RW[2000 + c];
            for (uint32_t i = lane; i < uint32_t(K) * POOL; i += G) pring(grp)[i] = 12.0f;
            for (uint32_t i = lane; i < 32; i += G) {
                s_cmd[grp][i] = 0.0f;
                a.commands[size_t(nn) * 32 + i] = 0.0f;
            }
            float* ring = a.sensors + size_t(nn) * 8 * PIX;
            for (uint32_t i = lane; i < 8 * PIX; i += G) ring[i] = 12.0f;
        }
        group_sync();
        if (ended)
            for (uint32_t i = lane; i < WORLD_WORDS; i += G) a.world[size_t(nn) * WORLD_WORDS + i] = world[i];
    }
    if constexpr (W > 1) {
        group_sync();
#pragma unroll
        for (int c = 0; c < 16; c++) r.hidden[c] = s_rh[grp][c];
    }
    if (live) {
        store_state(a.state, N, n, s, lane, G);
        store_run(a.run, N, n, r, lane, G);
    }
}

// navigation_training::validate_rollout (navigation_training.hpp:27-35): the
// lowest env whose task is not valid and ready (out[0]) and the lowest whose
// plant mass is not finite and positive (out[1]); 0xffffffff when none.  The
// caller fills out with 0xffffffff first.
__global__ __launch_bounds__(256) void validate_kernel(const MdnTaskState* __restrict__ tasks,
                                                       const MdnPhysicsParams* __restrict__ phys, uint32_t n,
                                                       uint32_t* __restrict__ out) {
    const uint32_t e = blockIdx.x * 256 + threadIdx.x;
    if (e >= n) return;
    const MdnTaskState& t = tasks[e];
    if (!(t.valid != 0u && t.generation_status == MDN_TASK_READY)) atomicMin(out, e);
    const float m = phys[e].mass;
    if (!(isfinite_f(m) && m > 0.0f)) atomicMin(out + 1, e);
}

}  // namespace nav

// ---------------------------------------------------------------- launchers
extern "C" {

hipError_t nav_launch_validate(const MdnTaskState* tasks, const MdnPhysicsParams* phys, uint32_t n, uint32_t* out,
                               hipStream_t stream) {
    hipError_t e = hipMemsetAsync(out, 0xff, 8, stream);
    if (e != hipSuccess || n == 0) return e;
    hipLaunchKernelGGL(nav::validate_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, tasks, phys, n, out);
    return hipGetLastError();
}

hipError_t nav_launch_episode(const nav::EpisodeArgs* a, hipStream_t stream) {
    if (a->cfg.n == 0) return hipSuccess;
    hipLaunchKernelGGL(nav::episode_kernel, dim3(a->cfg.n), dim3(64), 0, stream, *a);
    return hipGetLastError();
}

hipError_t nav_launch_reset(const nav::RolloutArgs* a, hipStream_t stream) {
    const uint32_t blocks = (a->cfg.n + 63) / 64;
    hipLaunchKernelGGL(nav::reset_kernel, dim3(blocks), dim3(64), 0, stream, *a);
    return hipGetLastError();
}

// Lanes per env G and pooled ring slots K are compile-time; K = sensor_delay+2
// rounded up to 2, 4 or 8.
// The 8-lane cases run four wavefronts per workgroup with the weights in LDS
// (32 envs, one workgroup per CU); with 4 or 8 slots the pooled ring lives
// in HBM (a.pool_ring).  16 and 4 lanes per env run one wavefront per
// workgroup with the weights in L1/L2.
// Split ticks (a->ext_means set) and 184-input actors are built for 8 lanes
// per env only.
hipError_t nav_launch_rollout(const nav::RolloutArgs* a, int lanes_per_env, int ring_slots, uint32_t actor_obs,
                              hipStream_t stream) {
    const bool dyn = a->env_phys != nullptr;
#define NAV_ROLLOUT_CASE_DYN(G, K, W, X, D, DYN)                                                                \
    if (lanes_per_env == G && ring_slots == K && (a->ext_means != nullptr) == X && actor_obs == D &&            \
        dyn == DYN) {                                                                                           \
        const uint32_t envs_per_block = 64 * W / G;                                                             \
        const uint32_t blocks = (a->cfg.n + envs_per_block - 1) / envs_per_block;                               \
        hipLaunchKernelGGL((nav::rollout_kernel<G, K, W, X, D, DYN>), dim3(blocks), dim3(64 * W), 0, stream, *a); \
        return hipGetLastError();                                                                               \
    }
#define NAV_ROLLOUT_CASE(G, K, W, X, D) NAV_ROLLOUT_CASE_DYN(G, K, W, X, D, false)
    constexpr uint32_t P = MDN_ACTOR_OBS_POOLED, H = MDN_ACTOR_OBS_PRIOR;
    // the Crazyflie plant as compile-time constants (the common plant of the
    // 8-lane instances with two ring slots, fused or split)
    const bool cf = !dyn && std::memcmp(&a->phys, &mdn::kCrazyflie, sizeof(MdnPhysicsParams)) == 0;
#define NAV_ROLLOUT_CASE_CF(G, K, W, X, D)                                                                     \
    if (cf && lanes_per_env == G && ring_slots == K && (a->ext_means != nullptr) == X && actor_obs == D) {     \
        const uint32_t blocks = (a->cfg.n + 64 * W / G - 1) / (64 * W / G);                                    \
        hipLaunchKernelGGL((nav::rollout_kernel<G, K, W, X, D, false, true>), dim3(blocks), dim3(64 * W), 0,   \
                           stream, *a);                                                                        \
        return hipGetLastError();                                                                              \
    }
    NAV_ROLLOUT_CASE_CF(8, 2, 4, false, P) NAV_ROLLOUT_CASE_CF(8, 4, 4, false, P)
    NAV_ROLLOUT_CASE_CF(8, 2, 4, false, H)
    NAV_ROLLOUT_CASE_CF(8, 2, 4, true, P) NAV_ROLLOUT_CASE_CF(8, 2, 4, true, H)
#undef NAV_ROLLOUT_CASE_CF
    NAV_ROLLOUT_CASE(8, 2, 4, false, P) NAV_ROLLOUT_CASE(8, 4, 4, false, P) NAV_ROLLOUT_CASE(8, 8, 4, false, P)
    NAV_ROLLOUT_CASE(16, 2, 1, false, P) NAV_ROLLOUT_CASE(16, 4, 1, false, P) NAV_ROLLOUT_CASE(16, 8, 1, false, P)
    NAV_ROLLOUT_CASE(4, 2, 1, false, P) NAV_ROLLOUT_CASE(4, 4, 1, false, P) NAV_ROLLOUT_CASE(4, 8, 1, false, P)
    NAV_ROLLOUT_CASE(8, 2, 4, true, P) NAV_ROLLOUT_CASE(8, 4, 4, true, P) NAV_ROLLOUT_CASE(8, 8, 4, true, P)
    NAV_ROLLOUT_CASE(8, 2, 4, false, H) NAV_ROLLOUT_CASE(8, 4, 4, false, H) NAV_ROLLOUT_CASE(8, 8, 4, false, H)
    NAV_ROLLOUT_CASE(8, 2, 4, true, H) NAV_ROLLOUT_CASE(8, 4, 4, true, H) NAV_ROLLOUT_CASE(8, 8, 4, true, H)
    // per-episode plants and navigation tasks: 8 lanes, the in-kernel policy,
    // one wavefront per workgroup (the per-env plant rows do not fit beside
    // the LDS-resident weights)
    NAV_ROLLOUT_CASE_DYN(8, 2, 1, false, P, true) NAV_ROLLOUT_CASE_DYN(8, 4, 1, false, P, true)
    NAV_ROLLOUT_CASE_DYN(8, 8, 1, false, P, true) NAV_ROLLOUT_CASE_DYN(8, 2, 1, false, H, true)
    NAV_ROLLOUT_CASE_DYN(8, 4, 1, false, H, true) NAV_ROLLOUT_CASE_DYN(8, 8, 1, false, H, true)
#undef NAV_ROLLOUT_CASE
#undef NAV_ROLLOUT_CASE_DYN
    return hipErrorInvalidValue;
}

}  // extern "C"

// ---------------------------------------------------------------- RAPTOR fixture
namespace nav {
// Each lane group runs RAPTOR from the initial hidden state over obs[steps][22]
// with the production group step (raptor_fixture, main.mm:74-77).
template <int G>
__global__ __launch_bounds__(64) void raptor_fixture_kernel(const float* __restrict__ RW, const float* __restrict__ obs,
                                                            uint32_t steps, uint32_t copies, float* __restrict__ actions,
                                                            float* __restrict__ hidden_out) {
    constexpr int E = 64 / G, U = 16 / G;
    __shared__ float s_x[E][17];
    __shared__ float s_h[E][17];
    const uint32_t lane = threadIdx.x % G, grp = threadIdx.x / G;
    const uint32_t copy = blockIdx.x * E + grp;
    const bool live = copy < copies;
    float hidden[16], hu[U];
#pragma unroll
    for (int j = 0; j < 16; j++) hidden[j] = RW[2000 + j];
#pragma unroll
    for (int j = 0; j < U; j++) hu[j] = RW[2000 + lane + G * j];
    for (uint32_t t = 0; t < steps; t++) {
        float mo[22];
#pragma unroll
        for (int j = 0; j < 22; j++) mo[j] = obs[t * 22 + j];
        float act[4];
        raptor_group<G>(RW, mo, hidden, hu, s_x[grp], s_h[grp], lane, live, act);
        if (live && lane == 0) {
            // the fixture reports the raw network output (raptor.hpp:51),
            // recomputed here without the clip
#pragma unroll
            for (int q = 0; q < 4; q++) {
                float val = RW[2080 + q];
#pragma unroll
                for (int col = 0; col < 16; col++) val = fma_f(RW[2016 + q * 16 + col], hidden[col], val);
                actions[(size_t(copy) * steps + t) * 4 + q] = val;
            }
        }
    }
    if (live && lane == 0)
        for (int j = 0; j < 16; j++) hidden_out[size_t(copy) * 16 + j] = hidden[j];
}
}  // namespace nav

extern "C" hipError_t nav_launch_raptor_fixture(const float* RW, const float* obs, uint32_t steps, uint32_t copies,
                                                float* actions, float* hidden, int lanes_per_env, hipStream_t st) {
    const uint32_t per = 64 / lanes_per_env;
    const dim3 grid((copies + per - 1) / per);
    if (lanes_per_env == 4) hipLaunchKernelGGL(nav::raptor_fixture_kernel<4>, grid, dim3(64), 0, st, RW, obs, steps, copies, actions, hidden);
    else if (lanes_per_env == 8) hipLaunchKernelGGL(nav::raptor_fixture_kernel<8>, grid, dim3(64), 0, st, RW, obs, steps, copies, actions, hidden);
    else if (lanes_per_env == 16) hipLaunchKernelGGL(nav::raptor_fixture_kernel<16>, grid, dim3(64), 0, st, RW, obs, steps, copies, actions, hidden);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}
