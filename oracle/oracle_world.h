/*
 * oracle_world.h — CPU oracle, part 1: scene geometry, plant and controller.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the checker for the HIP path: only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 * It restates, in plain scalar C++, the reference functions cited on each
 * definition; paths are relative to the reference repository.
 *
 * One deliberate restatement (applied identically in the HIP kernels): the
 * slab test of an axis-aligned box evaluates (-e-p)*(1/d) and (e-p)*(1/d)
 * where world.hpp:53 evaluates (-e-p)/d and (e-p)/d.  The reciprocal is taken
 * once per ray and axis; the bounds move by at most one rounding, and
 * tests/test_oracle_ref.py measures the depth difference against the
 * reference's own wray compiled from world.hpp.
 */
#ifndef MDNAV_ORACLE_WORLD_H
#define MDNAV_ORACLE_WORLD_H

#include <cstdint>
#include "mdnav_host.h"
#include "mdnav_math.h"
#include "mdnav_types.h"

namespace orc {
using namespace mdn;

struct V3 { float x, y, z; };
inline V3 v3(float x, float y, float z) { return {x, y, z}; }
inline V3 vadd(V3 a, V3 b) { return v3(a.x + b.x, a.y + b.y, a.z + b.z); }
inline V3 vsub(V3 a, V3 b) { return v3(a.x - b.x, a.y - b.y, a.z - b.z); }
inline V3 vmul(V3 a, float s) { return v3(a.x * s, a.y * s, a.z * s); }
inline float vdot(V3 a, V3 b) { return a.x * b.x + a.y * b.y + a.z * b.z; }
inline float vlen(V3 a) { return sqrt_f(vdot(a, a)); }
// world.hpp:25
inline V3 vnorm(V3 a) { return vmul(a, 1.0f / fmax_f(vlen(a), 1e-8f)); }

// world.hpp:32-41 — obstacle centre at time t (kind 3: bounded sinusoid).
inline V3 obstacle_center(const MdnObstacle& o, float t) {
    if (o.kind == 3) {
        const V3 velocity = v3(o.velocity[0], o.velocity[1], o.velocity[2]);
        const float speed = vlen(velocity), amplitude = o.size[1];
        if (speed <= 1e-8f || amplitude <= 1e-8f) return v3(o.center[0], o.center[1], o.center[2]);
        const float offset = amplitude * sin_f(t * speed / amplitude + o.size[2]) / speed;
        return vadd(v3(o.center[0], o.center[1], o.center[2]), vmul(velocity, offset));
    }
    return v3(o.center[0] + t * o.velocity[0], o.center[1] + t * o.velocity[1], o.center[2] + t * o.velocity[2]);
}

// world.hpp:42-47
inline float ray_sphere(V3 p, V3 d, V3 c, float r) {
    const V3 q = vsub(p, c);
    const float b = vdot(q, d), k = vdot(q, q) - r * r, disc = b * b - k;
    if (disc < 0) return 1000;
    const float lo = -b - sqrt_f(disc), hi = -b + sqrt_f(disc);
    return lo >= 0 ? lo : (hi >= 0 ? hi : 1000);
}

// Per-ray reciprocal direction used by the slab test.
struct RayInv { float inv[3]; bool parallel[3]; };
inline RayInv ray_inverse(V3 d) {
    RayInv r;
    const float dd[3] = {d.x, d.y, d.z};
    for (int j = 0; j < 3; j++) {
        r.parallel[j] = fabs_f(dd[j]) < 1e-8f;
        r.inv[j] = r.parallel[j] ? 0.0f : 1.0f / dd[j];
    }
    return r;
}

// world.hpp:48-57 (reciprocal form, see header comment).
inline float ray_box(V3 p, const RayInv& ri, V3 c, V3 extent) {
    float lo = -1e20f, hi = 1e20f;
    const float pp[3] = {p.x - c.x, p.y - c.y, p.z - c.z}, ee[3] = {extent.x, extent.y, extent.z};
    for (int j = 0; j < 3; j++) {
        if (ri.parallel[j]) {
            if (fabs_f(pp[j]) > ee[j]) return 1000;
        } else {
            const float a = (-ee[j] - pp[j]) * ri.inv[j], b = (ee[j] - pp[j]) * ri.inv[j];
            lo = fmax_f(lo, fmin_f(a, b));
            hi = fmin_f(hi, fmax_f(a, b));
        }
    }
    if (hi < fmax_f(lo, 0.0f)) return 1000;
    return lo >= 0 ? lo : hi;
}

// world.hpp:58-70
inline float ray_cylinder(V3 p, V3 d, V3 c, float r, float h) {
    const V3 q = vsub(p, c);
    const float a = d.x * d.x + d.y * d.y, b = q.x * d.x + q.y * d.y, k = q.x * q.x + q.y * q.y - r * r;
    float best = 1000;
    const float disc = b * b - a * k;
    if (a > 1e-10f && disc >= 0) {
        const float roots[2] = {(-b - sqrt_f(disc)) / a, (-b + sqrt_f(disc)) / a};
        for (int j = 0; j < 2; j++) {
            const float t = roots[j];
            if (t >= 0 && fabs_f(q.z + t * d.z) <= h) best = fmin_f(best, t);
        }
    }
    if (fabs_f(d.z) > 1e-8f)
        for (int sign = -1; sign <= 1; sign += 2) {
            const float t = (float(sign) * h - q.z) / d.z;
            const float x = q.x + t * d.x, y = q.y + t * d.y;
            if (t >= 0 && x * x + y * y <= r * r) best = fmin_f(best, t);
        }
    return best;
}

// world.hpp:71-83 — range of one ray: room box (x[-2,14], y[-5,5], z[0,5]),
// then every obstacle at `time`, clamped to [0, 12].
inline float ray_world(const MdnWorld& w, V3 p, V3 d, float time) {
    const RayInv ri = ray_inverse(d);
    float best = 12;
    best = fmin_f(best, ray_box(p, ri, v3(6, 0, 2.5f), v3(8, 5, 2.5f)));
    for (uint32_t i = 0; i < w.count; i++) {
        const MdnObstacle& o = w.obstacles[i];
        const V3 c = obstacle_center(o, time);
        float t = 1000;
        if (o.kind == 0) t = ray_box(p, ri, c, v3(o.size[0], o.size[1], o.size[2]));
        if (o.kind == 1 || o.kind == 3) t = ray_sphere(p, d, c, o.size[0]);
        if (o.kind == 2) t = ray_cylinder(p, d, c, o.size[0], o.size[2]);
        best = fmin_f(best, t);
    }
    return fmax_f(0.0f, best);
}

// world.hpp:84-99 — signed clearance of a 0.18 m body sphere.
inline float obstacle_distance(const MdnObstacle& o, V3 q) {
    if (o.kind == 1 || o.kind == 3) return vlen(q) - o.size[0];
    if (o.kind == 2) {
        const float a = sqrt_f(q.x * q.x + q.y * q.y) - o.size[0], b = fabs_f(q.z) - o.size[2];
        return sqrt_f(fmax_f(a, 0.0f) * fmax_f(a, 0.0f) + fmax_f(b, 0.0f) * fmax_f(b, 0.0f)) + fmin_f(fmax_f(a, b), 0.0f);
    }
    const V3 k = v3(fabs_f(q.x) - o.size[0], fabs_f(q.y) - o.size[1], fabs_f(q.z) - o.size[2]);
    return vlen(v3(fmax_f(k.x, 0.0f), fmax_f(k.y, 0.0f), fmax_f(k.z, 0.0f))) + fmin_f(fmax_f(k.x, fmax_f(k.y, k.z)), 0.0f);
}
inline float room_clearance(V3 p) {
    return fmin_f(fmin_f(p.x + 2, 14 - p.x), fmin_f(fmin_f(p.y + 5, 5 - p.y), fmin_f(p.z, 5 - p.z))) - 0.18f;
}
inline float clearance(const MdnWorld& w, V3 p, float time) {
    float best = room_clearance(p);
    for (uint32_t i = 0; i < w.count; i++) {
        const MdnObstacle& o = w.obstacles[i];
        const float distance = obstacle_distance(o, vsub(p, obstacle_center(o, time)));
        best = fmin_f(best, distance - 0.18f);
    }
    return best;
}

// sensor_profile.hpp:81-91 — unit ray of pixel k (row-major 20x16, row 0 up)
// for the profile's vertical half-tangent (0.75 legacy, 0.8 native).
inline V3 camera_ray(uint32_t pixel, float tan_v = MDN_SENSOR_TAN_V) {
    const uint32_t row = pixel / MDN_SENSOR_WIDTH, col = pixel % MDN_SENSOR_WIDTH;
    const float y = ((float(col) + 0.5f) / 20.0f * 2.0f - 1.0f) * MDN_SENSOR_TAN_H;
    const float z = ((float(row) + 0.5f) / 16.0f * 2.0f - 1.0f) * tan_v;
    return vnorm(v3(1.0f, -y, -z));
}

// ---- world generation: world.hpp:104-318 --------------------------------
// Where the reference passes several RNG draws as arguments of one call, the
// draws are sequenced left to right (the order clang gives the reference).
inline void world_add(MdnWorld& w, uint32_t kind, V3 c, V3 e, V3 v) {
    if (w.count >= 16) return;
    MdnObstacle& o = w.obstacles[w.count++];
    o.kind = kind;
    o.center[0] = c.x; o.center[1] = c.y; o.center[2] = c.z;
    o.size[0] = e.x; o.size[1] = e.y; o.size[2] = e.z;
    o.velocity[0] = v.x; o.velocity[1] = v.y; o.velocity[2] = v.z;
}
inline void world_add_box(MdnWorld& w, V3 c, V3 e) { world_add(w, 0, c, e, v3(0, 0, 0)); }
inline void world_add_table(MdnWorld& w, float x, float y, float hx, float hy, float top) {
    const float slab = 0.08f, underside = top - slab;
    world_add_box(w, v3(x, y, top), v3(hx, hy, slab));
    const float lx = hx - 0.12f, ly = hy - 0.12f, leg = 0.08f;
    const float lcz = underside * 0.5f, lhz = underside * 0.5f;
    world_add_box(w, v3(x - lx, y - ly, lcz), v3(leg, leg, lhz));
    world_add_box(w, v3(x - lx, y + ly, lcz), v3(leg, leg, lhz));
    world_add_box(w, v3(x + lx, y - ly, lcz), v3(leg, leg, lhz));
    world_add_box(w, v3(x + lx, y + ly, lcz), v3(leg, leg, lhz));
}
inline float route_y(const MdnWorld& w, float x, float distance) { return w.goal[1] * (x / distance); }
inline void world_add_doorway(MdnWorld& w, float wall_x, float gy, float gz, float hg, float hgz) {
    const float low_y = gy - hg, high_y = gy + hg, low_z = gz - hgz, high_z = gz + hgz, whx = 0.12f;
    world_add_box(w, v3(wall_x, (-5.0f + low_y) * 0.5f, 2.5f), v3(whx, (low_y + 5.0f) * 0.5f, 2.5f));
    world_add_box(w, v3(wall_x, (high_y + 5.0f) * 0.5f, 2.5f), v3(whx, (5.0f - high_y) * 0.5f, 2.5f));
    world_add_box(w, v3(wall_x, 0, low_z * 0.5f), v3(whx, 5.0f, low_z * 0.5f));
    world_add_box(w, v3(wall_x, 0, (high_z + 5.0f) * 0.5f), v3(whx, 5.0f, (5.0f - high_z) * 0.5f));
}
inline void gen_doorway(MdnWorld& w, uint32_t& rng, float distance) {
    const float wall_x = distance * (0.42f + 0.16f * urand(rng));
    const float rf = wall_x / distance;
    const float gy = w.goal[1] * rf + (urand(rng) - 0.5f) * 1.20f;
    const float hg = 0.40f + 0.30f * urand(rng);
    const float rz = 1.5f + (w.goal[2] - 1.5f) * rf;
    const float gz = rz + (urand(rng) - 0.5f) * 0.20f;
    const float hgz = 0.65f + 0.25f * urand(rng);
    world_add_doorway(w, wall_x, gy, gz, hg, hgz);
}
inline void gen_two_doorways(MdnWorld& w, uint32_t& rng, float distance) {
    for (uint32_t door = 0; door < 2; door++) {
        const float u0 = urand(rng);
        const float fraction = door == 0 ? 0.33f + 0.02f * (u0 - 0.5f) : 0.67f + 0.02f * (u0 - 0.5f);
        const float wall_x = distance * fraction;
        const float rf = wall_x / distance;
        const float gy = route_y(w, wall_x, distance) + (urand(rng) - 0.5f) * 1.00f;
        const float rz = 1.5f + (w.goal[2] - 1.5f) * rf;
        const float gz = rz + (urand(rng) - 0.5f) * 0.24f;
        const float hg = 0.40f + 0.30f * urand(rng);
        const float hgz = 0.65f + 0.25f * urand(rng);
        world_add_doorway(w, wall_x, gy, gz, hg, hgz);
    }
}
inline void gen_table_or_counter(MdnWorld& w, uint32_t& rng, float distance) {
    const float x = distance * (0.45f + 0.10f * urand(rng));
    const float y = route_y(w, x, distance) + (urand(rng) - 0.5f) * 0.20f;
    if (urand(rng) < 0.5f) {
        const float hx = 0.55f + 0.20f * urand(rng);
        const float hy = 0.75f + 0.20f * urand(rng);
        const float top = 1.55f + 0.50f * urand(rng);
        world_add_table(w, x, y, hx, hy, top);
    } else {
        const float hx = 0.60f + 0.20f * urand(rng);
        const float hy = 0.80f + 0.20f * urand(rng);
        const float height = 1.35f + 0.80f * urand(rng);
        world_add_box(w, v3(x, y, height * 0.5f), v3(hx, hy, height * 0.5f));
    }
}
inline void gen_mixed(MdnWorld& w, uint32_t& rng, float distance) {
    const float table_x = distance * (0.46f + 0.08f * urand(rng));
    const float table_y = route_y(w, table_x, distance) + (urand(rng) - 0.5f) * 0.16f;
    const float thx = 0.58f + 0.10f * urand(rng);
    const float thy = 0.76f + 0.10f * urand(rng);
    const float ttop = 1.62f + 0.42f * urand(rng);
    world_add_table(w, table_x, table_y, thx, thy, ttop);
    const float counter_x = distance * 0.22f;
    const float counter_y = route_y(w, counter_x, distance) - 1.30f;
    const float counter_h = 1.55f + 0.45f * urand(rng);
    world_add_box(w, v3(counter_x, counter_y, counter_h * 0.5f), v3(0.30f, 0.50f, counter_h * 0.5f));
    const float sphere_x = distance * 0.72f;
    const float sphere_y = route_y(w, sphere_x, distance) + 1.35f;
    const float sphere_r = 0.34f + 0.10f * urand(rng);
    const float sphere_z = 1.05f + 1.10f * urand(rng);
    const float sign = urand(rng) < 0.5f ? -1.0f : 1.0f;
    const float sphere_vy = sign * (0.18f + 0.16f * urand(rng));
    world_add(w, 1, v3(sphere_x, sphere_y, sphere_z), v3(sphere_r, sphere_r, sphere_r), v3(0, sphere_vy, 0));
    const float pole_r0 = 0.20f + 0.08f * urand(rng);
    const float pole_r1 = 0.20f + 0.08f * urand(rng);
    world_add(w, 2, v3(distance * 0.34f, route_y(w, distance * 0.34f, distance) + 2.05f, 2.5f), v3(pole_r0, pole_r0, 2.5f), v3(0, 0, 0));
    world_add(w, 2, v3(distance * 0.82f, route_y(w, distance * 0.82f, distance) - 2.05f, 2.5f), v3(pole_r1, pole_r1, 2.5f), v3(0, 0, 0));
    const float low_box_x = distance * 0.74f;
    const float low_box_y = route_y(w, low_box_x, distance) - 0.88f;
    world_add_box(w, v3(low_box_x, low_box_y, 0.48f), v3(0.34f, 0.30f, 0.48f));
}
inline void gen_threat_sphere(MdnWorld& w, uint32_t seed, uint32_t family) {
    const float drone_speed = 1.5f;
    uint32_t rng = seed ^ 0x9e3779b9u;
    if (rng == 0) rng = 1;
    const float lateral = (urand(rng) - 0.5f) * 0.20f;
    const float vertical = (urand(rng) - 0.5f) * 0.16f;
    const uint32_t speed_choice = xorshift(rng) % 3;
    const float threat_speed = speed_choice == 0 ? 0.5f : (speed_choice == 1 ? 1.0f : 2.0f);
    const float nominal_ttc = 0.7f + 0.8f * urand(rng);
    const float combined_radius = 0.18f + 0.35f;
    V3 center, velocity = v3(0, 0, 0);
    if (family == 10) {
        center = v3((drone_speed + threat_speed) * nominal_ttc + combined_radius, lateral, 1.5f + vertical);
        velocity.x = -threat_speed;
    } else {
        center = v3(drone_speed * nominal_ttc, -threat_speed * nominal_ttc + lateral, 1.5f + vertical);
        velocity.y = threat_speed;
    }
    w.goal[0] = 4.0f; w.goal[1] = 0.0f; w.goal[2] = 1.5f;
    world_add(w, 1, center, v3(0.35f, 0.35f, 0.35f), velocity);
}
inline float challenge_distance(float d) { return fmin_f(fmax_f(d, 3.0f), 10.0f); }
inline void gen_goal_span(MdnWorld& w, uint32_t& rng, float distance) {
    const float span = challenge_distance(distance);
    w.goal[0] = span * (0.90f + 0.10f * urand(rng));
    w.goal[1] = (urand(rng) - 0.5f) * 1.20f;
    w.goal[2] = 1.10f + 0.80f * urand(rng);
}
inline void gen_bent_hallway(MdnWorld& w, uint32_t& rng, float distance) {
    const float difficulty = urand(rng);
    gen_goal_span(w, rng, distance);
    const float wall_x = w.goal[0] * (0.24f + 0.04f * urand(rng));
    const float gap_x = w.goal[0] * (0.70f + 0.08f * difficulty);
    const float lane_width = 1.80f - 0.80f * difficulty;
    const float lane_edge = 5.0f - lane_width;
    const float wall_y = (-5.0f + lane_edge) * 0.5f;
    const float wall_half_y = (lane_edge + 5.0f) * 0.5f;
    world_add_box(w, v3(wall_x, wall_y, 2.5f), v3(0.15f, wall_half_y, 2.5f));
    world_add_box(w, v3((wall_x + gap_x) * 0.5f, lane_edge + 0.03f, 2.5f), v3((gap_x - wall_x) * 0.5f + 0.15f, 0.15f, 2.5f));
}
inline void gen_connected_rooms(MdnWorld& w, uint32_t& rng, float distance) {
    const float difficulty = urand(rng);
    gen_goal_span(w, rng, distance);
    const float wall_1 = w.goal[0] * (0.16f + 0.02f * urand(rng));
    const float wall_2 = w.goal[0] * 0.85f;
    const float gap_1 = -(0.60f + 0.80f * difficulty);
    const float gap_2 = +(0.60f + 0.80f * difficulty);
    const float gap_half = 0.85f - 0.30f * difficulty;
    const float gap_z = 1.50f;
    const float gap_half_z = 0.85f - 0.10f * difficulty;
    world_add_doorway(w, wall_1, gap_1, gap_z, gap_half, gap_half_z);
    world_add_doorway(w, wall_2, gap_2, gap_z, gap_half, gap_half_z);
    const float table_x = w.goal[0] * 0.50f;
    const float table_y = (urand(rng) - 0.5f) * 0.20f;
    const float table_half_x = fmin_f(0.45f, w.goal[0] * 0.06f);
    const float table_half_y = 0.60f + 0.20f * difficulty;
    const float table_top = 1.45f + 0.25f * difficulty;
    world_add_table(w, table_x, table_y, table_half_x, table_half_y, table_top);
    world_add_box(w, v3(w.goal[0] * 0.38f, 3.75f, 0.55f), v3(0.22f, 0.35f, 0.55f));
    world_add_box(w, v3(w.goal[0] * 0.50f, -3.80f, 0.80f), v3(0.25f, 0.35f, 0.80f));
    world_add_box(w, v3(w.goal[0] * 0.62f, 3.70f, 0.50f), v3(0.22f, 0.40f, 0.50f));
}
inline void gen_vertical_choices(MdnWorld& w, uint32_t& rng, float distance) {
    const float difficulty = urand(rng);
    gen_goal_span(w, rng, distance);
    const float low_x = w.goal[0] * (0.14f + 0.02f * (1.0f - difficulty));
    const float overhead_x = w.goal[0] * (0.46f + 0.02f * difficulty);
    const float choice_x = w.goal[0] * (0.76f + 0.02f * difficulty);
    const float low_top = 1.50f + 0.25f * difficulty;
    const float overhead_bottom = 2.80f - 0.20f * difficulty;
    const float choice_half_z = 0.10f + 0.05f * difficulty;
    world_add_box(w, v3(low_x, 0, low_top * 0.5f), v3(0.12f, 5.0f, low_top * 0.5f));
    const float overhead_half_z = (5.0f - overhead_bottom) * 0.5f;
    world_add_box(w, v3(overhead_x, 0, overhead_bottom + overhead_half_z), v3(0.12f, 5.0f, overhead_half_z));
    world_add_box(w, v3(choice_x, 0, 2.0f + choice_half_z), v3(0.10f, 5.0f, choice_half_z));
}
// world.hpp:293-298
inline uint32_t training_family(uint32_t family, uint32_t& rng) {
    if (family == 7) return xorshift(rng) % 7;
    if (family == 9 || family == 12) {
        const uint32_t choice = xorshift(rng) % 4;
        return choice < 2 ? 4 : (choice == 2 ? 5 : xorshift(rng) % 7);
    }
    if (family == 13) {
        const uint32_t choice = xorshift(rng) % 6;
        if (choice < 2) return 4;
        if (choice == 2) return 5;
        if (choice == 3) return xorshift(rng) % 7;
        return choice == 4 ? 10 : 11;
    }
    return family;
}
// Moving-threat mix (families MDN_FAMILY_MOVERS, _MOVERS_LONG, _COURSE; a
// workload of this library, not a reference generator).  Four kind-3
// bounded movers (world.hpp:26-41): radius U[0.2, 0.5] m, peak speed
// U[0.3, 1.5] m/s on a horizontal heading, amplitude U[0.5, 2] m, phase
// U[-pi, pi), centres along the route to `reach`.
inline void gen_movers(MdnWorld& w, uint32_t& rng, float reach) {
    for (int i = 0; i < 4; i++) {
        const float cx = 1.5f + urand(rng) * fmax_f(0.5f, reach - 2.5f);
        const float cy = (urand(rng) - 0.5f) * 5.0f;
        const float cz = 0.8f + urand(rng) * 1.6f;
        const float radius = 0.2f + 0.3f * urand(rng);
        const float speed = 0.3f + 1.2f * urand(rng);
        const float heading = 6.28318530718f * urand(rng);
        const float amplitude = 0.5f + 1.5f * urand(rng);
        const float phase = (urand(rng) - 0.5f) * 6.28318530718f;
        float sh, ch;
        sincos_f(heading, &sh, &ch);
        world_add(w, 3, v3(cx, cy, cz), v3(radius, amplitude, phase), v3(speed * ch, speed * sh, 0.0f));
    }
}
// The combined course of navigation_challenge_tasks.py:47-117 with xorshift
// draws: corridor walls with a side opening at 0.59 L (4 boxes), openings
// at 0.32 L and 0.68 L offset to alternate sides (4 boxes), a hanging beam
// at 0.5 L, and a bounded sphere of radius 0.28 m crossing at the side
// opening.  Start height 1.5 m (the reset's), goal (L, U[-0.2, 0.2], 1.5).
inline void gen_course(MdnWorld& w, uint32_t& rng) {
    const float length = 8.5f + 3.0f * urand(rng);
    const float yg = (urand(rng) - 0.5f) * 0.4f;
    const float z = 1.5f, width = 3.2f, cross = length * 0.59f;
    w.goal[0] = length; w.goal[1] = yg; w.goal[2] = z;
    for (int side = -1; side <= 1; side += 2) {
        const float y = float(side) * (width * 0.5f + 0.06f);
        const float spans[2][2] = {{-2.0f, cross - 0.7f}, {cross + 0.7f, 14.0f}};
        for (int k = 0; k < 2; k++) {
            const float lo = spans[k][0], hi = spans[k][1];
            world_add_box(w, v3((lo + hi) * 0.5f, y, 2.5f), v3((hi - lo) * 0.5f, 0.06f, 2.5f));
        }
    }
    const bool hard = urand(rng) < 0.5f;
    const float ug = urand(rng);
    const float gap = hard ? 0.85f + 0.35f * ug : 1.15f + 0.40f * ug;
    const float uo = urand(rng);
    const float offset = hard ? 0.65f + 0.20f * uo : 0.45f + 0.20f * uo;
    const float sign = urand(rng) < 0.5f ? -1.0f : 1.0f;
    for (int stage = 0; stage < 2; stage++) {
        const float x = length * (stage == 0 ? 0.32f : 0.68f);
        const float cy = sign * offset * (stage == 0 ? 1.0f : -1.0f);
        const float spans[2][2] = {{-width * 0.5f, cy - gap * 0.5f}, {cy + gap * 0.5f, width * 0.5f}};
        for (int k = 0; k < 2; k++) {
            const float lo = spans[k][0], hi = spans[k][1];
            world_add_box(w, v3(x, (lo + hi) * 0.5f, 2.5f), v3(0.12f, (hi - lo) * 0.5f, 2.5f));
        }
    }
    world_add_box(w, v3(length * 0.5f, 0.0f, 3.35f), v3(0.25f, width * 0.5f, 1.65f));
    const float us = urand(rng);
    const float speed = hard ? 0.65f + 0.35f * us : 0.35f + 0.30f * us;
    const float phase = -1.57079632679f + (urand(rng) - 0.5f) * 0.5f;
    const float dir = urand(rng) < 0.5f ? -1.0f : 1.0f;
    const float amplitude = 2.2f + 1.2f * urand(rng);
    world_add(w, 3, v3(cross, 0.0f, z), v3(0.28f, amplitude, phase), v3(0.0f, dir * speed, 0.0f));
}
// world.hpp:299-318
inline void generate_world(MdnWorld& w, uint32_t seed, uint32_t family, float distance) {
    uint32_t rng = seed ? seed : 1;
    w.seed = seed; w.family = family; w.count = family == 0 ? 0 : 8;
    w.goal[0] = distance;
    w.goal[1] = (urand(rng) - 0.5f) * 2;
    w.goal[2] = 1.5f + (urand(rng) - 0.5f) * 0.8f;
    for (int j = 0; j < 3; j++) w.wind[j] = 0;
    if (family == 4) { w.count = 0; gen_doorway(w, rng, distance); return; }
    if (family == 5) { w.count = 0; gen_table_or_counter(w, rng, distance); return; }
    if (family == 6) { w.count = 0; gen_mixed(w, rng, distance); return; }
    if (family == 8) { w.count = 0; gen_two_doorways(w, rng, distance); return; }
    if (family == 10 || family == 11) { w.count = 0; gen_threat_sphere(w, seed, family); return; }
    if (family == 14) { w.count = 0; gen_bent_hallway(w, rng, distance); return; }
    if (family == 15) { w.count = 0; gen_connected_rooms(w, rng, distance); return; }
    if (family == 16) { w.count = 0; gen_vertical_choices(w, rng, distance); return; }
    if (family == MDN_FAMILY_COURSE) { w.count = 0; gen_course(w, rng); return; }
    const bool mover_world = family == MDN_FAMILY_MOVERS || family == MDN_FAMILY_MOVERS_LONG;
    float reach = distance;
    if (family == MDN_FAMILY_MOVERS_LONG) { reach = 8.0f + 5.0f * urand(rng); w.goal[0] = reach; }
    for (uint32_t i = 0; i < 16; i++) {
        MdnObstacle& o = w.obstacles[i];
        o.kind = family == 2 ? 2 : (family == 3 ? 1 : 0);
        o.center[0] = 1.2f + urand(rng) * fmax_f(0.1f, reach - 2.2f);
        o.center[1] = (urand(rng) - 0.5f) * 7;
        o.center[2] = family == 2 ? 2.5f : 0.6f + urand(rng) * 3;
        o.size[0] = 0.2f + urand(rng) * 0.35f;
        o.size[1] = 0.3f + urand(rng) * 0.55f;
        o.size[2] = family == 2 ? 2.5f : 0.2f + urand(rng) * 0.75f;
        o.velocity[0] = 0;
        o.velocity[1] = family == 3 ? (urand(rng) - 0.5f) * 0.8f : 0;
        o.velocity[2] = 0;
    }
    if (mover_world) gen_movers(w, rng, reach);  // slots 8-11
}

// ---- L2F plant: physics.hpp:44-179 --------------------------------------
inline void cross3(const float a[3], const float b[3], float out[3]) {
    out[0] = a[1] * b[2] - a[2] * b[1];
    out[1] = a[2] * b[0] - a[0] * b[2];
    out[2] = a[0] * b[1] - a[1] * b[0];
}
inline void rotate_body_to_world(const float q[4], const float v[3], float out[3]) {
    const float tx = 2.0f * (q[2] * v[2] - q[3] * v[1]);
    const float ty = 2.0f * (q[3] * v[0] - q[1] * v[2]);
    const float tz = 2.0f * (q[1] * v[1] - q[2] * v[0]);
    out[0] = v[0] + q[0] * tx + q[2] * tz - q[3] * ty;
    out[1] = v[1] + q[0] * ty + q[3] * tx - q[1] * tz;
    out[2] = v[2] + q[0] * tz + q[1] * ty - q[2] * tx;
}
inline void derivative(const MdnPhysicsParams& p, const MdnPhysicsState& s, const float setpoint[4],
                       const float wind[3], MdnPhysicsState& d) {
    float thrust[3] = {0, 0, 0}, torque[3] = {0, 0, 0};
    for (int r = 0; r < 4; ++r) {
        const float speed = s.rpm[r];
        const float* c = &p.rotor_thrust_coefficients[3 * r];
        const float magnitude = c[0] + c[1] * speed + c[2] * speed * speed;
        float rt[3];
        const float* direction = &p.rotor_thrust_directions[3 * r];
        for (int i = 0; i < 3; ++i) {
            rt[i] = direction[i] * magnitude;
            thrust[i] += rt[i];
            torque[i] += p.rotor_torque_directions[3 * r + i] * magnitude * p.rotor_torque_constants[r];
        }
        float arm[3];
        cross3(&p.rotor_positions[3 * r], rt, arm);
        for (int i = 0; i < 3; ++i) torque[i] += arm[i];
    }
    for (int i = 0; i < 3; ++i) d.position[i] = s.linear_velocity[i];
    const float* q = s.orientation_wxyz;
    const float* w = s.angular_velocity_body;
    d.orientation_wxyz[0] = -q[1] * w[0] - q[2] * w[1] - q[3] * w[2];
    d.orientation_wxyz[1] = q[0] * w[0] + q[2] * w[2] - q[3] * w[1];
    d.orientation_wxyz[2] = q[0] * w[1] + q[3] * w[0] - q[1] * w[2];
    d.orientation_wxyz[3] = q[0] * w[2] + q[1] * w[1] - q[2] * w[0];
    for (int i = 0; i < 4; ++i) d.orientation_wxyz[i] *= 0.5f;
    rotate_body_to_world(q, thrust, d.linear_velocity);
    for (int i = 0; i < 3; ++i)
        d.linear_velocity[i] = d.linear_velocity[i] / p.mass + p.gravity_world[i] + wind[i] / p.mass;
    float am[3] = {0, 0, 0};
    for (int row = 0; row < 3; ++row)
        for (int col = 0; col < 3; ++col) am[row] += p.inertia[3 * row + col] * w[col];
    float gyro[3];
    cross3(w, am, gyro);
    for (int i = 0; i < 3; ++i) am[i] = torque[i] - gyro[i];
    for (int row = 0; row < 3; ++row) {
        d.angular_velocity_body[row] = 0.0f;
        for (int col = 0; col < 3; ++col) d.angular_velocity_body[row] += p.inertia_inverse[3 * row + col] * am[col];
    }
    for (int r = 0; r < 4; ++r) {
        const float tau = setpoint[r] >= s.rpm[r] ? p.rotor_time_constants_rising[r] : p.rotor_time_constants_falling[r];
        d.rpm[r] = (setpoint[r] - s.rpm[r]) / tau;
    }
}
inline void add_scaled(const MdnPhysicsState& s, const MdnPhysicsState& d, float scale, MdnPhysicsState& out) {
    const float* a = &s.position[0];
    const float* b = &d.position[0];
    float* o = &out.position[0];
    for (int i = 0; i < 17; ++i) o[i] = a[i] + scale * b[i];
}
inline void physics_step(const MdnPhysicsState& state, const float action[4], const float wind[3],
                         const MdnPhysicsParams& p, MdnPhysicsState& next) {
    float setpoint[4];
    const float half = (p.action_max - p.action_min) * 0.5f;
    for (int i = 0; i < 4; ++i) {
        float a = action[i];
        if (a < -1.0f) a = -1.0f;
        if (a > 1.0f) a = 1.0f;
        setpoint[i] = a * half + p.action_min + half;
    }
    MdnPhysicsState k1, k2, k3, k4, temp;
    derivative(p, state, setpoint, wind, k1);
    add_scaled(state, k1, 0.5f * p.dt, temp);
    derivative(p, temp, setpoint, wind, k2);
    add_scaled(state, k2, 0.5f * p.dt, temp);
    derivative(p, temp, setpoint, wind, k3);
    add_scaled(state, k3, p.dt, temp);
    derivative(p, temp, setpoint, wind, k4);
    const float* s = &state.position[0];
    const float* a1 = &k1.position[0];
    const float* a2 = &k2.position[0];
    const float* a3 = &k3.position[0];
    const float* a4 = &k4.position[0];
    float* o = &next.position[0];
    // a + 2b as one fma (2b is exact): the same value, one rounding
    for (int i = 0; i < 17; ++i) o[i] = s[i] + p.dt * (std::fma(2.0f, a3[i], std::fma(2.0f, a2[i], a1[i])) + a4[i]) / 6.0f;
    float* q = next.orientation_wxyz;
    const float norm = sqrt_f(q[0] * q[0] + q[1] * q[1] + q[2] * q[2] + q[3] * q[3]);
    for (int i = 0; i < 4; ++i) q[i] /= norm;
    for (int i = 0; i < 3; ++i) {
        if (next.position[i] < -p.position_limit) next.position[i] = -p.position_limit;
        if (next.position[i] > p.position_limit) next.position[i] = p.position_limit;
        if (next.linear_velocity[i] < -p.velocity_limit) next.linear_velocity[i] = -p.velocity_limit;
        if (next.linear_velocity[i] > p.velocity_limit) next.linear_velocity[i] = p.velocity_limit;
        if (next.angular_velocity_body[i] < -p.angular_velocity_limit) next.angular_velocity_body[i] = -p.angular_velocity_limit;
        if (next.angular_velocity_body[i] > p.angular_velocity_limit) next.angular_velocity_body[i] = p.angular_velocity_limit;
    }
    for (int i = 0; i < 4; ++i) {
        if (next.rpm[i] < p.action_min) next.rpm[i] = p.action_min;
        if (next.rpm[i] > p.action_max) next.rpm[i] = p.action_max;
    }
}

// ---- RAPTOR inner loop: raptor.hpp:42-97 --------------------------------
// Dense and GRU dot products are fma chains from the bias, inputs ascending
// (the same canonical form as the policy networks).
inline void raptor_reset(const MdnRaptorWeights& w, float hidden[16]) {
    for (int i = 0; i < 16; i++) hidden[i] = w.initial_hidden_state[i];
}
inline void raptor_forward(const MdnRaptorWeights& w, const float obs[22], float hidden[16], float action[4]) {
    float x[16];
    for (int row = 0; row < 16; ++row) {
        float value = w.input_bias[row];
        for (int col = 0; col < 22; ++col) value = fma_f(w.input_weights[row * 22 + col], obs[col], value);
        x[row] = max_f(value, 0.0f);
    }
    float ig[48], hg[48];
    for (int row = 0; row < 48; ++row) {
        float iv = w.gru_input_bias[row], hv = w.gru_hidden_bias[row];
        for (int col = 0; col < 16; ++col) {
            iv = fma_f(w.gru_input_weights[row * 16 + col], x[col], iv);
            hv = fma_f(w.gru_hidden_weights[row * 16 + col], hidden[col], hv);
        }
        ig[row] = iv;
        hg[row] = hv;
    }
    float nh[16];
    for (int i = 0; i < 16; ++i) {
        const float reset = sigmoid_f(ig[i] + hg[i]);
        const float update = sigmoid_f(ig[16 + i] + hg[16 + i]);
        const float candidate = tanh_f(ig[32 + i] + reset * hg[32 + i]);
        nh[i] = (1.0f - update) * candidate + update * hidden[i];
    }
    for (int i = 0; i < 16; ++i) hidden[i] = nh[i];
    for (int row = 0; row < 4; ++row) {
        float value = w.output_bias[row];
        for (int col = 0; col < 16; ++col) value = fma_f(w.output_weights[row * 16 + col], hidden[col], value);
        action[row] = value;
    }
}
inline void raptor_clip(float a[4]) {
    for (int i = 0; i < 4; i++) a[i] = max_f(-1.0f, min_f(1.0f, a[i]));
}

// sim.metal:43-48 == cpu_reference.hpp:82-87
inline void rotation(const float q[4], float r[9]) {
    const float w = q[0], x = q[1], y = q[2], z = q[3];
    r[0] = 1 - 2 * (y * y + z * z); r[1] = 2 * (x * y - w * z); r[2] = 2 * (x * z + w * y);
    r[3] = 2 * (x * y + w * z); r[4] = 1 - 2 * (x * x + z * z); r[5] = 2 * (y * z - w * x);
    r[6] = 2 * (x * z - w * y); r[7] = 2 * (y * z + w * x); r[8] = 1 - 2 * (x * x + y * y);
}

// sim.metal:49 == cpu_reference.hpp:76-80
inline float sim_normal(uint32_t& rng) {
    const float u = max_f(urand(rng), 1e-7f);
    const float v = urand(rng);
    return sqrt_f(-2.0f * log_f(u)) * cos_f(6.28318530718f * v);
}

} // namespace orc

#endif
