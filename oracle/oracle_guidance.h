// oracle_guidance.h — CPU restatement of the geometry-prior guidance
// (guidance.hpp:21-194): the 3-value hint appended to a 184-input actor's
// observation (ppo.hpp:30, 77; sim.metal:226 == cpu_reference.hpp:353-375).
//
// Test infrastructure: only tests/, __graft_entry__.smoke() and bench.py's
// CPU baseline use it.  Written over the shared math (mdnav_math.h: sqrt_f is
// correctly rounded, log_f is this project's own log), so it matches the GPU
// bit for bit and the reference's guidance.hpp to the ulps of std::log.
#pragma once

#include <cstdint>

#include "mdnav_math.h"

namespace orc {
using namespace mdn;

// guidance.hpp:21-26: direction of pooled cell (row, col) of the 8x10 grid
inline void nav_ray(uint32_t row, uint32_t col, float tan_v, float* d) {
    const float y = 0.9f - 0.2f * float(col), z = (0.875f - 0.25f * float(row)) * tan_v;
    const float inv = 1.0f / sqrt_f(1.0f + y * y + z * z);
    d[0] = inv;
    d[1] = y * inv;
    d[2] = z * inv;
}

// guidance.hpp:27-34: nearest range in the 3x3 neighbourhood, row-major
inline float nav_min3x3(const float* range, uint32_t row, uint32_t col) {
    float nearest = 12.0f;
    for (int dr = -1; dr <= 1; dr++)
        for (int dc = -1; dc <= 1; dc++) {
            const int r = int(row) + dr, c = int(col) + dc;
            if (r >= 0 && r < 8 && c >= 0 && c < 10) nearest = fmin_f(nearest, range[r * 10 + c]);
        }
    return nearest;
}

inline float nav_atanh(float x) { return 0.5f * log_f((1.0f + x) / (1.0f - x)); }

// guidance.hpp:55-63: closing-speed risk of the 3x3 neighbourhood of (row, col)
inline float nav_temporal_risk(const float* current, const float* previous, const float* vel, float sensor_dt,
                               float tan_v, uint32_t row, uint32_t col) {
    float risk = 0.0f;
    if (!(sensor_dt > 1e-4f)) return risk;
    for (int dr = -1; dr <= 1; dr++)
        for (int dc = -1; dc <= 1; dc++) {
            const int r = int(row) + dr, c = int(col) + dc;
            if (r < 0 || r >= 8 || c < 0 || c >= 10) continue;
            const uint32_t k = uint32_t(r * 10 + c);
            const float old = previous[k], now = current[k];
            if (old < 11.9f && now < 11.9f) {
                float ray[3];
                nav_ray(uint32_t(r), uint32_t(c), tan_v, ray);
                const float unexpected = (old - now) / fmax_f(sensor_dt, 1e-3f) -
                                         (vel[0] * ray[0] + vel[1] * ray[1] + vel[2] * ray[2]);
                if (unexpected > 0.5f) risk = fmax_f(risk, fmin_f(0.20f * unexpected, 1.0f));
            }
        }
    return risk;
}

// guidance.hpp:38-98 (memory-less prior)
inline void nav_guidance(const float* current, const float* previous, const float* goal_body_unit, float goal_distance,
                         const float* vel, float sensor_dt, float tan_v, float* hint) {
    const float gnorm = sqrt_f(goal_body_unit[0] * goal_body_unit[0] + goal_body_unit[1] * goal_body_unit[1] +
                               goal_body_unit[2] * goal_body_unit[2]);
    if (gnorm < 1e-6f || goal_distance < 0.05f) {
        hint[0] = hint[1] = hint[2] = 0.0f;
        return;
    }
    const float goal[3] = {goal_body_unit[0] / gnorm, goal_body_unit[1] / gnorm, goal_body_unit[2] / gnorm};
    const float speed = sqrt_f(vel[0] * vel[0] + vel[1] * vel[1] + vel[2] * vel[2]);
    const float stop_margin = 0.28f + speed * fmax_f(sensor_dt, 0.0f) + 0.25f * speed * speed;
    float best_score = -1e20f, best_dir[3] = {1, 0, 0}, best_range = 0;
    float goal_cell_dot = -1e20f;
    uint32_t goal_row = 0, goal_col = 0;
    for (uint32_t row = 0; row < 8; row++)
        for (uint32_t col = 0; col < 10; col++) {
            float d[3];
            nav_ray(row, col, tan_v, d);
            const float alignment = d[0] * goal[0] + d[1] * goal[1] + d[2] * goal[2];
            const float nearby = nav_min3x3(current, row, col);
            const float risk = nav_temporal_risk(current, previous, vel, sensor_dt, tan_v, row, col);
            const float safe_range = fmax_f(nearby - risk, 0.0f);
            const float score = 1.4f * alignment + 0.12f * fmin_f(safe_range, 6.0f);
            if (score > best_score) {
                best_score = score;
                best_dir[0] = d[0]; best_dir[1] = d[1]; best_dir[2] = d[2];
                best_range = safe_range;
            }
            if (alignment > goal_cell_dot) {
                goal_cell_dot = alignment;
                goal_row = row;
                goal_col = col;
            }
        }
    const float max_speed = 1.6f;
    const float desired_speed = fmin_f(max_speed, sqrt_f(4.0f * fmax_f(goal_distance - 0.28f, 0.0f)));
    const float direct_range = fmax_f(nav_min3x3(current, goal_row, goal_col), 0.0f);
    float direction[3] = {best_dir[0], best_dir[1], best_dir[2]}, available = best_range;
    if (goal[0] > 0.0f && direct_range > stop_margin + 0.25f * desired_speed * desired_speed) {
        direction[0] = goal[0]; direction[1] = goal[1]; direction[2] = goal[2];
        available = direct_range;
    }
    const float after_stop = fmax_f(available - stop_margin - 0.15f, 0.0f);
    const float command_speed = fmin_f(desired_speed, sqrt_f(4.0f * after_stop));
    const float fraction = fmin_f(0.8f, command_speed * 0.5f);
    if (direct_range < 1.2f && available > direct_range + 0.25f) {
        const float advance = fmax_f(0.05f, fmin_f(1.0f, (direct_range - 0.25f) / 0.95f));
        direction[0] *= advance;
        const float norm = sqrt_f(direction[0] * direction[0] + direction[1] * direction[1] + direction[2] * direction[2]);
        for (int i = 0; i < 3; i++) direction[i] /= fmax_f(norm, 1e-6f);
    }
    for (int i = 0; i < 3; i++) hint[i] = nav_atanh(fraction * direction[i]);
}

// guidance.hpp:100-107 (capture age off, the reference's default)
inline float nav_memory_point_radius(float range, float history_age) {
    const float age = fmax_f(history_age, 0.0f) + 0.0f;
    return 0.20f + 0.015f * range + 0.15f * age;
}

// guidance.hpp:109-147: first swept-sphere contact along a body-frame
// direction from the remembered range hits and ego poses.
inline float nav_memory_clearance(const float* direction, const float* range_ring, const float* pose_ring,
                                  const float* current_pose, uint32_t latest_frame, uint32_t valid_frames,
                                  float sensor_dt, float tan_v) {
    float nearest = 3.0f;
    for (uint32_t back = 0; back < valid_frames && back < 8; back++) {
        const uint32_t frame = (latest_frame + 8u - back) % 8u;
        const float* old_pose = pose_ring + frame * 12;
        const float* ranges = range_ring + frame * 320;
        const float age = float(back) * fmax_f(sensor_dt, 0.0f);
        for (uint32_t row = 0; row < 8; row++)
            for (uint32_t col = 0; col < 10; col++) {
                const uint32_t px = row * 2 * 20 + col * 2;
                uint32_t hit = px;
                float range = ranges[px];
                const uint32_t pixels[3] = {px + 1, px + 20, px + 21};
                for (int j = 0; j < 3; j++)
                    if (ranges[pixels[j]] < range) { range = ranges[pixels[j]]; hit = pixels[j]; }
                if (range <= 0.01f || range >= 11.9f) continue;
                const float ry = 1.0f - (float(hit % 20) + .5f) / 10.0f, rz = tan_v * (1.0f - (float(hit / 20) + .5f) / 8.0f);
                const float inv = 1.0f / sqrt_f(1 + ry * ry + rz * rz);
                const float ray[3] = {inv, ry * inv, rz * inv};
                const float wx = old_pose[3] * ray[0] + old_pose[4] * ray[1] + old_pose[5] * ray[2];
                const float wy = old_pose[6] * ray[0] + old_pose[7] * ray[1] + old_pose[8] * ray[2];
                const float wz = old_pose[9] * ray[0] + old_pose[10] * ray[1] + old_pose[11] * ray[2];
                const float dx = old_pose[0] + range * wx - current_pose[0];
                const float dy = old_pose[1] + range * wy - current_pose[1];
                const float dz = old_pose[2] + range * wz - current_pose[2];
                const float x = current_pose[3] * dx + current_pose[6] * dy + current_pose[9] * dz;
                const float y = current_pose[4] * dx + current_pose[7] * dy + current_pose[10] * dz;
                const float z = current_pose[5] * dx + current_pose[8] * dy + current_pose[11] * dz;
                const float along = x * direction[0] + y * direction[1] + z * direction[2];
                const float radius = nav_memory_point_radius(range, age);
                if (along <= 0.0f || along > 3.0f + radius) continue;
                const float lateral2 = fmax_f(x * x + y * y + z * z - along * along, 0.0f);
                const float radius2 = radius * radius;
                if (lateral2 < radius2) nearest = fmin_f(nearest, fmax_f(along - sqrt_f(radius2 - lateral2), 0.0f));
            }
    }
    return nearest;
}

// guidance.hpp:152-194 (history-aware prior, clearances computed directly as
// in the CPU reference's call, cpu_reference.hpp:369-372)
inline void nav_guidance_memory(const float* current, const float* previous, const float* goal_body_unit,
                                float goal_distance, const float* vel, float sensor_dt, float tan_v,
                                const float* range_ring, const float* pose_ring, const float* current_pose,
                                uint32_t latest_frame, uint32_t valid_frames, float* hint) {
    const float gnorm = sqrt_f(goal_body_unit[0] * goal_body_unit[0] + goal_body_unit[1] * goal_body_unit[1] +
                               goal_body_unit[2] * goal_body_unit[2]);
    if (gnorm < 1e-6f || goal_distance < 0.05f) {
        hint[0] = hint[1] = hint[2] = 0.0f;
        return;
    }
    const float goal[3] = {goal_body_unit[0] / gnorm, goal_body_unit[1] / gnorm, goal_body_unit[2] / gnorm};
    const float speed = sqrt_f(vel[0] * vel[0] + vel[1] * vel[1] + vel[2] * vel[2]);
    const float stop_margin = 0.28f + speed * fmax_f(sensor_dt, 0.0f) + 0.25f * speed * speed;
    float goal_cell_dot = -1e20f;
    uint32_t goal_row = 0, goal_col = 0;
    for (uint32_t row = 0; row < 8; row++)
        for (uint32_t col = 0; col < 10; col++) {
            float d[3];
            nav_ray(row, col, tan_v, d);
            const float a = d[0] * goal[0] + d[1] * goal[1] + d[2] * goal[2];
            if (a > goal_cell_dot) { goal_cell_dot = a; goal_row = row; goal_col = col; }
        }
    const float desired_speed = fmin_f(1.6f, sqrt_f(4.0f * fmax_f(goal_distance - 0.28f, 0.0f)));
    float best_score = -1e20f, best_free = 0.0f, best_dir[3] = {1, 0, 0};
    for (uint32_t candidate = 0; candidate < 85; candidate++) {
        float d[3];
        uint32_t row = goal_row, col = goal_col;
        if (candidate < 80) {
            row = candidate / 10;
            col = candidate % 10;
            nav_ray(row, col, tan_v, d);
        } else if (candidate == 80) {
            d[0] = goal[0]; d[1] = goal[1]; d[2] = goal[2];
        } else {
            d[0] = 0;
            d[1] = candidate >= 83 ? (candidate == 83 ? 1.0f : -1.0f) : 0;
            d[2] = candidate < 83 ? (candidate == 81 ? 1.0f : -1.0f) : 0;
        }
        float sweep[3] = {1.2f * d[0] + 0.35f * vel[0], 1.2f * d[1] + 0.35f * vel[1], 1.2f * d[2] + 0.35f * vel[2]};
        const float sweep_norm = sqrt_f(sweep[0] * sweep[0] + sweep[1] * sweep[1] + sweep[2] * sweep[2]);
        for (int j = 0; j < 3; j++) sweep[j] /= fmax_f(sweep_norm, 1e-6f);
        float free = nav_memory_clearance(sweep, range_ring, pose_ring, current_pose, latest_frame, valid_frames,
                                          sensor_dt, tan_v);
        const float observed = nav_min3x3(current, row, col);
        if (candidate < 81) free = fmin_f(free, observed);
        const float temporal_risk = nav_temporal_risk(current, previous, vel, sensor_dt, tan_v, row, col);
        free = fmax_f(free - temporal_risk, 0.0f);
        const float alignment = d[0] * goal[0] + d[1] * goal[1] + d[2] * goal[2];
        const float required = stop_margin + 0.15f + desired_speed * desired_speed * .25f;
        const float score = 1.4f * alignment + 0.20f * fmin_f(free, 3.0f) -
                            (free < required ? 3.0f * (required - free) / required : 0.0f);
        if (score > best_score) {
            best_score = score;
            best_free = free;
            best_dir[0] = d[0]; best_dir[1] = d[1]; best_dir[2] = d[2];
        }
    }
    const bool goal_in_fov = goal[0] > 0.0f && fabs_f(goal[1]) <= goal[0] && fabs_f(goal[2]) <= tan_v * goal[0];
    const float after_stop = fmax_f(best_free - stop_margin - 0.15f, 0.0f);
    float command_speed = fmin_f(desired_speed, sqrt_f(4.0f * after_stop));
    if (!goal_in_fov) command_speed = fmin_f(command_speed, 0.25f);
    const float fraction = fmin_f(0.8f, command_speed * 0.5f);
    for (int i = 0; i < 3; i++) hint[i] = nav_atanh(fraction * best_dir[i]);
}

}  // namespace orc
