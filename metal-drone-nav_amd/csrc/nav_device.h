// nav_device.h — device functions of the environment step for gfx950.
//
// Register-resident state, one env per lane group.  Arithmetic follows the
// reference expressions term by term (no re-association, contraction off) so
// the device and the CPU oracle round identically; file:line cites the
// reference function each block follows.
#pragma once

#include <hip/hip_runtime.h>

#include "mdnav_math.h"
#include "mdnav_plant.h"
#include "mdnav_types.h"

namespace nav {
using namespace mdn;

constexpr uint32_t PIX = MDN_SENSOR_PIXELS;
constexpr uint32_t POOL = MDN_POOLED_FEATURES;
constexpr uint32_t OBS = MDN_ACTOR_OBS_POOLED;
constexpr uint32_t COBS = MDN_CRITIC_OBS;
constexpr uint32_t HID = MDN_HIDDEN;
constexpr float LOG_TWO_PI = 1.8378770664093453f;

// Word offsets of SimRun (main.mm:454-460); the run block is stored as
// struct-of-arrays run[word][env].
enum RunWord : uint32_t {
    RW_HIDDEN = 0, RW_MOTORS = 16, RW_PREV_NAV = 20, RW_DESIRED_VEL = 24, RW_YAW = 27, RW_RNG = 28,
    RW_STEPS = 29, RW_PATH = 30, RW_ELAPSED = 31, RW_PEAK_SPEED = 32, RW_MIN_CLEARANCE = 33,
    RW_INITIAL_DISTANCE = 34, RW_SUCCESSES = 35, RW_COLLISIONS = 36, RW_TIMEOUTS = 37, RW_EPISODES = 38,
    RW_SUCCESS_TIME = 39, RW_TOTAL_PATH = 40, RW_TOTAL_ELAPSED = 41, RW_FINAL_PROGRESS = 42, RW_REF_POS = 43,
    RW_COUNT = 46
};
constexpr uint32_t STATE_WORDS = 17;
constexpr uint32_t WORLD_WORDS = 169;
constexpr uint32_t RAPTOR_WORDS = sizeof(MdnRaptorWeights) / sizeof(float);

struct State { float p[3], q[4], v[3], w[3], rpm[4]; };

struct Run {
    float hidden[16], motors[4], prev_nav[4], desired_vel[3], yaw;
    uint32_t rng, steps;
    float path, elapsed, peak_speed, min_clearance, initial_distance;
    uint32_t successes, collisions, timeouts, episodes;
    float success_time, total_path, total_elapsed, final_progress, ref_pos[3];
};
static_assert(sizeof(Run) == RW_COUNT * 4, "Run block");
static_assert(sizeof(State) == STATE_WORDS * 4, "State block");

// ---------------------------------------------------------------- RNG
// world.hpp:30-31
__device__ __forceinline__ uint32_t xs(uint32_t& s) { s ^= s << 13; s ^= s >> 17; s ^= s << 5; return s; }
__device__ __forceinline__ float ur(uint32_t& s) { return float(xs(s) >> 8) * (1.0f / 16777216.0f); }
// sim.metal:49
__device__ __forceinline__ float normal_draw(uint32_t& rng) {
    const float u = max_f(ur(rng), 1e-7f);
    const float v = ur(rng);
    return sqrt_f(-2.0f * log_f(u)) * cos_f(6.28318530718f * v);
}

// ---------------------------------------------------------------- geometry
struct V { float x, y, z; };
__device__ __forceinline__ V mk(float x, float y, float z) { V r; r.x = x; r.y = y; r.z = z; return r; }
__device__ __forceinline__ float dot3(V a, V b) { return a.x * b.x + a.y * b.y + a.z * b.z; }
__device__ __forceinline__ float len3(V a) { return sqrt_f(dot3(a, a)); }
__device__ __forceinline__ V sub3(V a, V b) { return mk(a.x - b.x, a.y - b.y, a.z - b.z); }

// Obstacle record as laid out in WWorld (world.hpp:28): kind, centre, size, velocity.
__device__ __forceinline__ V obstacle_center(const float* o, float t) {
    const uint32_t kind = float_bits(o[0]);
    if (kind == 3u) {  // world.hpp:33-38
        const V vel = mk(o[7], o[8], o[9]);
        const float speed = len3(vel), amplitude = o[5];
        if (speed <= 1e-8f || amplitude <= 1e-8f) return mk(o[1], o[2], o[3]);
        const float offset = amplitude * sin_f(t * speed / amplitude + o[6]) / speed;
        return mk(o[1] + vel.x * offset, o[2] + vel.y * offset, o[3] + vel.z * offset);
    }
    return mk(o[1] + t * o[7], o[2] + t * o[8], o[3] + t * o[9]);  // world.hpp:40
}

// world.hpp:42-47
__device__ __forceinline__ float hit_sphere(V p, V d, V c, float r) {
    const V q = sub3(p, c);
    const float b = dot3(q, d), k = dot3(q, q) - r * r, disc = b * b - k;
    if (disc < 0) return 1000;
    const float lo = -b - sqrt_f(disc), hi = -b + sqrt_f(disc);
    return lo >= 0 ? lo : (hi >= 0 ? hi : 1000);
}

// Slab test of world.hpp:48-57 with the per-ray reciprocal (1/d computed
// once per ray; the reference divides per box).
struct Slab { float inv[3]; bool par[3]; };
__device__ __forceinline__ Slab make_slab(V d) {
    Slab s;
    const float dd[3] = {d.x, d.y, d.z};
#pragma unroll
    for (int j = 0; j < 3; j++) {
        s.par[j] = fabs_f(dd[j]) < 1e-8f;
        s.inv[j] = s.par[j] ? 0.0f : 1.0f / dd[j];
    }
    return s;
}
__device__ __forceinline__ float hit_box(V p, const Slab& sl, V c, V e) {
    float lo = -1e20f, hi = 1e20f;
    const float pp[3] = {p.x - c.x, p.y - c.y, p.z - c.z}, ee[3] = {e.x, e.y, e.z};
#pragma unroll
    for (int j = 0; j < 3; j++) {
        if (sl.par[j]) {
            if (fabs_f(pp[j]) > ee[j]) return 1000;
        } else {
            const float a = (-ee[j] - pp[j]) * sl.inv[j], b = (ee[j] - pp[j]) * sl.inv[j];
            lo = fmax_f(lo, fmin_f(a, b));
            hi = fmin_f(hi, fmax_f(a, b));
        }
    }
    if (hi < fmax_f(lo, 0.0f)) return 1000;
    return lo >= 0 ? lo : hi;
}
// world.hpp:58-70
__device__ __noinline__ float hit_cylinder(V p, V d, V c, float r, float h) {
    const V q = sub3(p, c);
    const float a = d.x * d.x + d.y * d.y, b = q.x * d.x + q.y * d.y, k = q.x * q.x + q.y * q.y - r * r;
    float best = 1000;
    const float disc = b * b - a * k;
    if (a > 1e-10f && disc >= 0) {
        const float r0 = (-b - sqrt_f(disc)) / a, r1 = (-b + sqrt_f(disc)) / a;
        if (r0 >= 0 && fabs_f(q.z + r0 * d.z) <= h) best = fmin_f(best, r0);
        if (r1 >= 0 && fabs_f(q.z + r1 * d.z) <= h) best = fmin_f(best, r1);
    }
    if (fabs_f(d.z) > 1e-8f)
        for (int sign = -1; sign <= 1; sign += 2) {
            const float t = (float(sign) * h - q.z) / d.z;
            const float x = q.x + t * d.x, y = q.y + t * d.y;
            if (t >= 0 && x * x + y * y <= r * r) best = fmin_f(best, t);
        }
    return best;
}

// world.hpp:71-83 — obstacles in LDS (`world` = WWorld words), centres for
// the current time precomputed in `centers`.
__device__ __forceinline__ float cast_ray(const float* world, const float* centers, uint32_t count, V p, V d) {
    const Slab sl = make_slab(d);
    float best = 12;
    best = fmin_f(best, hit_box(p, sl, mk(6, 0, 2.5f), mk(8, 5, 2.5f)));
    for (uint32_t i = 0; i < count; i++) {
        const float* o = world + 10 * i;
        const uint32_t kind = float_bits(o[0]);
        const V c = mk(centers[3 * i], centers[3 * i + 1], centers[3 * i + 2]);
        float t = 1000;
        if (kind == 0u) t = hit_box(p, sl, c, mk(o[4], o[5], o[6]));
        else if (kind == 1u || kind == 3u) t = hit_sphere(p, d, c, o[4]);
        else if (kind == 2u) t = hit_cylinder(p, d, c, o[4], o[6]);
        best = fmin_f(best, t);
    }
    return fmax_f(0.0f, best);
}

// Fast path of cast_ray for a world of up to 8 axis-aligned boxes when no
// ray direction component is below the slab epsilon.  Per env and frame the
// constants (-e - pp) and (e - pp) of world.hpp:53 are formed once (same
// operations, hoisted out of the ray loop) into a slab table in LDS; per ray
// only the products with 1/d and the interval updates remain.  Inside the
// slab the hardware min/max may differ from the select form only in the sign
// of a zero, which the final fmax(0, best) of world.hpp:82 maps to +0, and
// the minimum of hit values that are never NaN does not depend on their
// order, so depths are bit-identical to cast_ray.
// Table words: slab 0 the room, slab 1 + i box i, 6 words each
// [A0 A1 A2 B0 B1 B2]; then the ray origin (3), the camera rotation (9) and
// the strip masks of the boxes (2 words, BOX_TABLE_STRIPS).
constexpr uint32_t BOX_TABLE_ORIGIN = 54, BOX_TABLE_ROT = 57, BOX_TABLE_STRIPS = 66, BOX_TABLE_WORDS = 68;
__device__ __forceinline__ void box_slab(const float* world, const float* centers, uint32_t i, V p, float (&A)[3],
                                         float (&B)[3]) {
    if (i == 0) {  // the room
        const float pr[3] = {p.x - 6.0f, p.y - 0.0f, p.z - 2.5f}, er[3] = {8.0f, 5.0f, 2.5f};
#pragma unroll
        for (int j = 0; j < 3; j++) { A[j] = -er[j] - pr[j]; B[j] = er[j] - pr[j]; }
        return;
    }
    const float* o = world + 10 * (i - 1);
    const float* c = centers + 3 * (i - 1);
    const float pp[3] = {p.x - c[0], p.y - c[1], p.z - c[2]};
#pragma unroll
    for (int j = 0; j < 3; j++) { A[j] = -o[4 + j] - pp[j]; B[j] = o[4 + j] - pp[j]; }
}

// Vertical strips of the depth frame (4 of its 20 columns each, 5 strips)
// whose rays can reach box [A, B] (coordinates relative to the ray origin)
// at a hit value below 12, as a 5-bit mask.  R is the camera rotation
// (row-major, world = R camera).  Camera rays are (1, -y, -z) normalised with
// |y| <= 0.95 tan_h and |z| <= 0.9375 tan_v at the pixel centres, so the rays of a strip
// lie in the wedge between the planes through its outer columns (the
// frame's rows and columns follow the camera rays of the sim's setup).  A box is
// left out of a strip only when one of those planes (or the image's top,
// bottom or back plane) separates it from the wedge with a gap above 1e-3 m,
// or when all of it lies beyond 12.01 m.  Rounding moves a slab test's
// interval ends by about 1e-6 m (relative 2^-24 of distances under 20 m, and
// of a rotation within 1e-6 of orthonormal), so such a box yields a miss or a
// value of at least 12 for every ray of the strip, and leaving it out does
// not change the depth.  The mask depends only on comparisons of finite
// values, so the hardware min/max (whose treatment of signed zeros differs
// from fmin_f's) gives the same mask.
__device__ __forceinline__ uint32_t box_strips(const float (&A)[3], const float (&B)[3], const float* R, float tan_v) {
    const float gap = 2e-3f;  // plane normals below have length <= 1.7
    float d2 = 0.0f;
#pragma unroll
    for (int j = 0; j < 3; j++) {
        const float c = __builtin_fminf(__builtin_fmaxf(0.0f, A[j]), B[j]);
        d2 += c * c;
    }
    if (d2 > 12.01f * 12.01f) return 0u;
    const float f[3] = {R[0], R[3], R[6]}, l[3] = {R[1], R[4], R[7]}, u[3] = {R[2], R[5], R[8]};
    // smallest value of n . x over the box
    auto support = [&](const float (&n)[3]) {
        float m = 0.0f;
#pragma unroll
        for (int j = 0; j < 3; j++) m += __builtin_fminf(n[j] * A[j], n[j] * B[j]);
        return m;
    };
    const float tv = 0.9375f * tan_v;  // |z| of the outer pixel rows
    {
        const float behind[3] = {-f[0], -f[1], -f[2]};
        const float top[3] = {-tv * f[0] - u[0], -tv * f[1] - u[1], -tv * f[2] - u[2]};
        const float bottom[3] = {-tv * f[0] + u[0], -tv * f[1] + u[1], -tv * f[2] + u[2]};
        if (support(behind) > gap || support(top) > gap || support(bottom) > gap) return 0u;
    }
    uint32_t mask = 0;
#pragma unroll
    for (uint32_t st = 0; st < 5; st++) {
        // ray ratio Y/X = -y(col), decreasing with the column
        const float r_hi = -((float(4 * st) + 0.5f) / 20.0f * 2.0f - 1.0f) * MDN_SENSOR_TAN_H;
        const float r_lo = -((float(4 * st + 3) + 0.5f) / 20.0f * 2.0f - 1.0f) * MDN_SENSOR_TAN_H;
        const float left[3] = {-r_hi * f[0] + l[0], -r_hi * f[1] + l[1], -r_hi * f[2] + l[2]};
        const float right[3] = {r_lo * f[0] - l[0], r_lo * f[1] - l[1], r_lo * f[2] - l[2]};
        if (!(support(left) > gap || support(right) > gap)) mask |= 1u << st;
    }
    return mask;
}
__device__ __forceinline__ bool boxes_only(const float* world, uint32_t count) {
    if (count > 8) return false;
    bool ok = true;
    for (uint32_t i = 0; i < count; i++) ok = ok && float_bits(world[10 * i]) == 0u;
    return ok;
}
__device__ __forceinline__ float slab_fast(const float (&A)[3], const float (&B)[3], const float (&inv)[3]) {
    float a = A[0] * inv[0], b = B[0] * inv[0];
    float lo = __builtin_fminf(a, b), hi = __builtin_fmaxf(a, b);
#pragma unroll
    for (int j = 1; j < 3; j++) {
        a = A[j] * inv[j];
        b = B[j] * inv[j];
        lo = __builtin_fmaxf(lo, __builtin_fminf(a, b));
        hi = __builtin_fminf(hi, __builtin_fmaxf(a, b));
    }
    return hi < __builtin_fmaxf(lo, 0.0f) ? 1000.0f : (lo >= 0 ? lo : hi);
}
// 1/d by the hardware reciprocal (v_rcp_f32) and one Newton step.  Over all
// 2^32 floats this equals the correctly rounded 1.0f / d for every finite d
// whose reciprocal is a normal number (|d| <= 2^126); the ray components here
// satisfy 1e-8 <= |d| <= 1.
__device__ __forceinline__ float recip_rn(float d) {
    const float y = __builtin_amdgcn_rcpf(d);
    return __builtin_fmaf(__builtin_fmaf(-d, y, 1.0f), y, y);
}
// Depth along d (every component at least the slab epsilon in magnitude)
// through an env's slab table: the room (row 0) and the boxes whose bits are
// set in the wavefront-uniform strip mask m (row i + 1 for bit i); the
// minimum of hit values, as cast_ray forms it for a boxes-only world.
__device__ __forceinline__ float strip_depth(const float (&SA)[9][3], const float (&SB)[9][3], V d, uint32_t m) {
    const float inv[3] = {recip_rn(d.x), recip_rn(d.y), recip_rn(d.z)};
    float best = __builtin_fminf(12.0f, slab_fast(SA[0], SB[0], inv));
#pragma unroll
    for (int i = 0; i < 8; i++)
        if ((m >> i) & 1u) best = __builtin_fminf(best, slab_fast(SA[i + 1], SB[i + 1], inv));
    return fmax_f(0.0f, best);
}
// Strip-culled cast of any world (boxes, spheres, bounded movers and capped
// cylinders; up to 16 obstacles), the wavefront casting one env's frame at a
// time as for boxes.  Per env and frame the env's lane group tabulates every
// obstacle with the per-obstacle constants of world.hpp:42-70, formed with
// the reference's operations (box: -e - pp and e - pp; sphere: q = p - c and
// q.q - r*r; cylinder: q, q.x^2 + q.y^2 - r*r, half height, r*r), and marks
// the 4-column strips its bounding box can reach (box_strips).  Per ray only
// the strip's obstacles are tested, by kind, with the operations of
// cast_ray, so each hit value is cast_ray's.
// A strip leaves out an obstacle only when a plane separates its bounding box
// from every ray of the strip by more than 2e-3 m, or when it lies beyond
// 12.01 m.  For a box that gives a miss or a value of at least 12 (above).
// For a sphere or cylinder of radius r the exact discriminant of such a ray is
// below -(0.004 r + 4e-6), while its fp32 rounding error is at most about
// 4e-5 (terms up to 12.5^2 = 156, a few ulps of 2^-23 each), so the computed
// discriminant stays negative when r >= 0.05 m; the cap test's point lies
// at least 2e-3 m outside the cap disk, again above its rounding error.
// Worlds with a smaller radius take the per-lane cast below.
// Table words: room slab 0-5, obstacle i at 6 + 6 i, then the ray origin,
// the camera rotation, strip masks (bit 16 (st % 2) + i of word st / 2) and
// two kind bits per obstacle (0 box, 1 sphere, 2 cylinder).
constexpr uint32_t STRIP_TABLE_ORIGIN = 102, STRIP_TABLE_ROT = 105, STRIP_TABLE_MASKS = 114,
                   STRIP_TABLE_KINDS = 117, STRIP_TABLE_WORDS = 118;
constexpr float STRIP_MIN_RADIUS = 0.05f;
__device__ __forceinline__ bool strip_castable(const float* world, uint32_t count) {
    if (count > 16) return false;
    bool ok = true;
    for (uint32_t i = 0; i < count; i++) {
        const uint32_t kind = float_bits(world[10 * i]);
        ok = ok && kind <= 3u && (kind == 0u || world[10 * i + 4] >= STRIP_MIN_RADIUS);
    }
    return ok;
}
// Obstacle i's table entry `e` (6 words) for origin p, its kind code and its
// bounding box relative to p (A = low corner, B = high corner).
__device__ __forceinline__ uint32_t strip_entry(const float* world, const float* centers, uint32_t i, V p, float* e,
                                                float (&A)[3], float (&B)[3]) {
    const float* o = world + 10 * i;
    const uint32_t kind = float_bits(o[0]);
    const V c = mk(centers[3 * i], centers[3 * i + 1], centers[3 * i + 2]);
    const float pp[3] = {p.x - c.x, p.y - c.y, p.z - c.z};
    if (kind == 0u) {  // world.hpp:53
#pragma unroll
        for (int j = 0; j < 3; j++) { A[j] = -o[4 + j] - pp[j]; B[j] = o[4 + j] - pp[j]; e[j] = A[j]; e[3 + j] = B[j]; }
        return 0u;
    }
    const V q = sub3(p, c);
    const float r = o[4];
    const float ext[3] = {r, r, kind == 2u ? o[6] : r};
#pragma unroll
    for (int j = 0; j < 3; j++) { A[j] = -ext[j] - pp[j]; B[j] = ext[j] - pp[j]; }
    e[0] = q.x; e[1] = q.y; e[2] = q.z;
    if (kind == 2u) {  // world.hpp:60
        e[3] = q.x * q.x + q.y * q.y - r * r;
        e[4] = o[6];
        e[5] = r * r;
        return 2u;
    }
    e[3] = dot3(q, q) - r * r;  // world.hpp:43 (kinds 1 and 3)
    return 1u;
}
// Depth along d (every component at least the slab epsilon in magnitude)
// over the room (RA, RB) and the obstacles of the wavefront-uniform strip
// mask m16 of the env table et; kinds holds two bits per obstacle.  The next
// entry's words are read while the current obstacle is tested.
__device__ __forceinline__ float strip_depth_mixed(const float* et, V d, uint32_t m16, uint32_t kinds,
                                                   const float (&RA)[3], const float (&RB)[3]) {
    const float inv[3] = {recip_rn(d.x), recip_rn(d.y), recip_rn(d.z)};
    float best = __builtin_fminf(12.0f, slab_fast(RA, RB, inv));
    const float a = d.x * d.x + d.y * d.y;
    const bool caps = fabs_f(d.z) > 1e-8f;
    uint32_t m = m16;
    float cur[6] = {0, 0, 0, 0, 0, 0};
    uint32_t ci = m ? uint32_t(__builtin_ctz(m)) : 0u;
    if (m) {
#pragma unroll
        for (int j = 0; j < 6; j++) cur[j] = et[6 + 6 * ci + j];
    }
    while (m) {
        m &= m - 1u;
        const uint32_t ni = m ? uint32_t(__builtin_ctz(m)) : ci;
        float nxt[6];
#pragma unroll
        for (int j = 0; j < 6; j++) nxt[j] = et[6 + 6 * ni + j];
        const uint32_t kind = (kinds >> (2u * ci)) & 3u;
        float t;
        if (kind == 0u) {
            const float A[3] = {cur[0], cur[1], cur[2]}, B[3] = {cur[3], cur[4], cur[5]};
            t = slab_fast(A, B, inv);
        } else if (kind == 1u) {  // hit_sphere (world.hpp:42-47)
            const V q = mk(cur[0], cur[1], cur[2]);
            const float b = dot3(q, d), disc = b * b - cur[3];
            const float root = sqrt_f(disc);
            const float lo = -b - root, hi = -b + root;
            t = disc < 0 ? 1000.0f : (lo >= 0 ? lo : (hi >= 0 ? hi : 1000.0f));
        } else {  // hit_cylinder (world.hpp:58-70)
            const V q = mk(cur[0], cur[1], cur[2]);
            const float k = cur[3], h = cur[4], rr = cur[5];
            const float b = q.x * d.x + q.y * d.y;
            const float disc = b * b - a * k;
            t = 1000.0f;
            if (a > 1e-10f && disc >= 0) {
                const float r0 = (-b - sqrt_f(disc)) / a, r1 = (-b + sqrt_f(disc)) / a;
                if (r0 >= 0 && fabs_f(q.z + r0 * d.z) <= h) t = fmin_f(t, r0);
                if (r1 >= 0 && fabs_f(q.z + r1 * d.z) <= h) t = fmin_f(t, r1);
            }
            if (caps)
                for (int sign = -1; sign <= 1; sign += 2) {
                    const float tc = (float(sign) * h - q.z) / d.z;
                    const float x = q.x + tc * d.x, y = q.y + tc * d.y;
                    if (tc >= 0 && x * x + y * y <= rr) t = fmin_f(t, tc);
                }
        }
        best = __builtin_fminf(best, t);
        ci = ni;
#pragma unroll
        for (int j = 0; j < 6; j++) cur[j] = nxt[j];
    }
    return fmax_f(0.0f, best);
}

// Fast path of cast_ray for worlds of up to 16 boxes, 8 spheres (kinds 1 and
// 3) and 8 capped cylinders when no ray direction component is below the slab
// epsilon.  Per env and frame the obstacles are tabulated in the env's LDS
// scratch row by kind, with every per-obstacle constant of world.hpp:42-70
// (q = p - c, q.q - r*r, r*r, the slab bounds -e - pp and e - pp) formed
// once with the reference's operations; per ray only the ray-dependent terms
// remain and the loops are branch-free with trip counts uniform over the
// wavefront (the largest count of each kind among its envs; slots past an
// env's own count are ignored).  Each obstacle's hit value is the one
// cast_ray computes, and the minimum of hit values that are never NaN and
// never negative does not depend on their order (a zero may change sign,
// which the final fmax(0, best) maps to +0), so depths are bit-identical.
constexpr uint32_t MIX_MAX_SPHERES = 8, MIX_MAX_CYLINDERS = 8;
// Table words for wave-wide counts: boxes (6 each), spheres (4), cylinders (6).
__device__ __forceinline__ uint32_t mix_words(uint32_t nb, uint32_t ns, uint32_t nc) { return 6 * nb + 4 * ns + 6 * nc; }
struct MixCounts { uint32_t nb, ns, nc; };
__device__ __forceinline__ bool mix_counts(const float* world, uint32_t count, MixCounts& m) {
    m.nb = m.ns = m.nc = 0;
    bool ok = count <= 16;
    for (uint32_t i = 0; i < count && i < 16; i++) {
        const uint32_t kind = float_bits(world[10 * i]);
        m.nb += kind == 0u;
        m.ns += kind == 1u || kind == 3u;
        m.nc += kind == 2u;
        ok = ok && kind <= 3u;
    }
    return ok && m.ns <= MIX_MAX_SPHERES && m.nc <= MIX_MAX_CYLINDERS;
}
// Writes the env's table for wave-wide counts (NB, NS, NC); lane `lane` of the
// env's G-lane group takes obstacles lane, lane + G, ...  `centers` holds the
// obstacle centres at the frame's time.
__device__ __forceinline__ void mix_table(const float* world, const float* centers, uint32_t count, V p, uint32_t NB,
                                          uint32_t NS, uint32_t lane, uint32_t G, float* tbl) {
    for (uint32_t i = lane; i < count; i += G) {
        const float* o = world + 10 * i;
        const uint32_t kind = float_bits(o[0]);
        const bool sph = kind == 1u || kind == 3u;
        uint32_t rank = 0;
        for (uint32_t j = 0; j < i; j++) {
            const uint32_t kj = float_bits(world[10 * j]);
            rank += sph ? (kj == 1u || kj == 3u) : kj == kind;
        }
        const V c = mk(centers[3 * i], centers[3 * i + 1], centers[3 * i + 2]);
        if (kind == 0u) {  // world.hpp:53: -e - pp and e - pp per axis
            float* e = tbl + 6 * rank;
            const float pp[3] = {p.x - c.x, p.y - c.y, p.z - c.z};
#pragma unroll
            for (int j = 0; j < 3; j++) { e[j] = -o[4 + j] - pp[j]; e[3 + j] = o[4 + j] - pp[j]; }
        } else if (sph) {  // world.hpp:43: q and q.q - r*r
            float* e = tbl + 6 * NB + 4 * rank;
            const V q = sub3(p, c);
            e[0] = q.x; e[1] = q.y; e[2] = q.z;
            e[3] = dot3(q, q) - o[4] * o[4];
        } else {  // world.hpp:60: q, q.x^2 + q.y^2 - r*r, half height, r*r
            float* e = tbl + 6 * NB + 4 * NS + 6 * rank;
            const V q = sub3(p, c);
            const float r = o[4];
            e[0] = q.x; e[1] = q.y; e[2] = q.z;
            e[3] = q.x * q.x + q.y * q.y - r * r;
            e[4] = o[6];
            e[5] = r * r;
        }
    }
}
__device__ __forceinline__ float cast_ray_mixed(const float (&RA)[3], const float (&RB)[3], const float* tbl,
                                                const MixCounts& own, uint32_t NB, uint32_t NS, uint32_t NC, V d) {
    const float inv[3] = {recip_rn(d.x), recip_rn(d.y), recip_rn(d.z)};
    float best = __builtin_fminf(12.0f, slab_fast(RA, RB, inv));
    for (uint32_t i = 0; i < NB; i++) {
        const float* e = tbl + 6 * i;
        const float A[3] = {e[0], e[1], e[2]}, B[3] = {e[3], e[4], e[5]};
        const float t = slab_fast(A, B, inv);
        best = __builtin_fminf(best, i < own.nb ? t : 1000.0f);
    }
    const float* sp = tbl + 6 * NB;
    for (uint32_t i = 0; i < NS; i++) {  // hit_sphere (world.hpp:42-47)
        const float* e = sp + 4 * i;
        const V q = mk(e[0], e[1], e[2]);
        const float b = dot3(q, d), disc = b * b - e[3];
        const float root = sqrt_f(disc);
        const float lo = -b - root, hi = -b + root;
        const float t = disc < 0 ? 1000.0f : (lo >= 0 ? lo : (hi >= 0 ? hi : 1000.0f));
        best = __builtin_fminf(best, i < own.ns ? t : 1000.0f);
    }
    const float* cy = sp + 4 * NS;
    const float a = d.x * d.x + d.y * d.y;
    const bool caps = fabs_f(d.z) > 1e-8f;
    for (uint32_t i = 0; i < NC; i++) {  // hit_cylinder (world.hpp:58-70)
        const float* e = cy + 6 * i;
        const V q = mk(e[0], e[1], e[2]);
        const float h = e[4], rr = e[5];
        const float b = q.x * d.x + q.y * d.y;
        float t = 1000;
        const float disc = b * b - a * e[3];
        if (a > 1e-10f && disc >= 0) {
            const float r0 = (-b - sqrt_f(disc)) / a, r1 = (-b + sqrt_f(disc)) / a;
            if (r0 >= 0 && fabs_f(q.z + r0 * d.z) <= h) t = fmin_f(t, r0);
            if (r1 >= 0 && fabs_f(q.z + r1 * d.z) <= h) t = fmin_f(t, r1);
        }
        if (caps)
            for (int sign = -1; sign <= 1; sign += 2) {
                const float tc = (float(sign) * h - q.z) / d.z;
                const float x = q.x + tc * d.x, y = q.y + tc * d.y;
                if (tc >= 0 && x * x + y * y <= rr) t = fmin_f(t, tc);
            }
        best = __builtin_fminf(best, i < own.nc ? t : 1000.0f);
    }
    return fmax_f(0.0f, best);
}
// cast_ray_mixed for the four rays of a pooled 2x2 block at once: each table
// entry is read from LDS once for the four rays, and the four rays' chains
// are independent.  Every ray needs all direction components >= 1e-8.
// Data-dependent branches of world.hpp:42-70 are selects here: both sides
// are evaluated and the taken side's value kept, which is the same value.
__device__ __forceinline__ void cast_block_mixed(const float (&RA)[3], const float (&RB)[3], const float* tbl,
                                                 const MixCounts& own, uint32_t NB, uint32_t NS, uint32_t NC,
                                                 const V (&d)[4], float (&out)[4]) {
    float inv[4][3], best[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        inv[r][0] = recip_rn(d[r].x); inv[r][1] = recip_rn(d[r].y); inv[r][2] = recip_rn(d[r].z);
        best[r] = __builtin_fminf(12.0f, slab_fast(RA, RB, inv[r]));
    }
    for (uint32_t i = 0; i < NB; i++) {
        const float* e = tbl + 6 * i;
        const float A[3] = {e[0], e[1], e[2]}, B[3] = {e[3], e[4], e[5]};
        const bool live = i < own.nb;
#pragma unroll
        for (int r = 0; r < 4; r++) best[r] = __builtin_fminf(best[r], live ? slab_fast(A, B, inv[r]) : 1000.0f);
    }
    const float* sp = tbl + 6 * NB;
    for (uint32_t i = 0; i < NS; i++) {  // hit_sphere (world.hpp:42-47)
        const float* e = sp + 4 * i;
        const V q = mk(e[0], e[1], e[2]);
        const float k = e[3];
        const bool live = i < own.ns;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float b = dot3(q, d[r]), disc = b * b - k;
            const float root = sqrt_f(disc);
            const float lo = -b - root, hi = -b + root;
            const float t = disc < 0 ? 1000.0f : (lo >= 0 ? lo : (hi >= 0 ? hi : 1000.0f));
            best[r] = __builtin_fminf(best[r], live ? t : 1000.0f);
        }
    }
    const float* cy = sp + 4 * NS;
    float a[4];
    bool caps[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        a[r] = d[r].x * d[r].x + d[r].y * d[r].y;
        caps[r] = fabs_f(d[r].z) > 1e-8f;
    }
    for (uint32_t i = 0; i < NC; i++) {  // hit_cylinder (world.hpp:58-70)
        const float* e = cy + 6 * i;
        const V q = mk(e[0], e[1], e[2]);
        const float k = e[3], h = e[4], rr = e[5];
        const bool live = i < own.nc;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float b = q.x * d[r].x + q.y * d[r].y;
            const float disc = b * b - a[r] * k;
            const bool side = a[r] > 1e-10f && disc >= 0;
            const float root = sqrt_f(disc);
            const float r0 = (-b - root) / a[r], r1 = (-b + root) / a[r];
            float t = 1000;
            t = side && r0 >= 0 && fabs_f(q.z + r0 * d[r].z) <= h ? fmin_f(t, r0) : t;
            t = side && r1 >= 0 && fabs_f(q.z + r1 * d[r].z) <= h ? fmin_f(t, r1) : t;
#pragma unroll
            for (int sign = -1; sign <= 1; sign += 2) {
                const float tc = (float(sign) * h - q.z) / d[r].z;
                const float x = q.x + tc * d[r].x, y = q.y + tc * d[r].y;
                t = caps[r] && tc >= 0 && x * x + y * y <= rr ? fmin_f(t, tc) : t;
            }
            best[r] = __builtin_fminf(best[r], live ? t : 1000.0f);
        }
    }
#pragma unroll
    for (int r = 0; r < 4; r++) out[r] = fmax_f(0.0f, best[r]);
}

// Largest value of a wave-uniform-call argument over the 64 lanes.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) v = max(v, uint32_t(__shfl_xor(int(v), off, 64)));
    return __builtin_amdgcn_readfirstlane(v);
}

// world.hpp:84-99
__device__ __forceinline__ float room_clearance(V p) {
    return fmin_f(fmin_f(p.x + 2, 14 - p.x), fmin_f(fmin_f(p.y + 5, 5 - p.y), fmin_f(p.z, 5 - p.z))) - 0.18f;
}
__device__ __forceinline__ float obstacle_clearance(const float* o, V p, float time) {
    const uint32_t kind = float_bits(o[0]);
    const V q = sub3(p, obstacle_center(o, time));
    float distance;
    if (kind == 1u || kind == 3u) distance = len3(q) - o[4];
    else if (kind == 2u) {
        const float a = sqrt_f(q.x * q.x + q.y * q.y) - o[4], b = fabs_f(q.z) - o[6];
        distance = sqrt_f(fmax_f(a, 0.0f) * fmax_f(a, 0.0f) + fmax_f(b, 0.0f) * fmax_f(b, 0.0f)) + fmin_f(fmax_f(a, b), 0.0f);
    } else {
        const V k = mk(fabs_f(q.x) - o[4], fabs_f(q.y) - o[5], fabs_f(q.z) - o[6]);
        distance = len3(mk(fmax_f(k.x, 0.0f), fmax_f(k.y, 0.0f), fmax_f(k.z, 0.0f))) + fmin_f(fmax_f(k.x, fmax_f(k.y, k.z)), 0.0f);
    }
    return distance - 0.18f;
}
__device__ __forceinline__ float clearance_at(const float* world, uint32_t count, V p, float time) {
    float best = room_clearance(p);
    for (uint32_t i = 0; i < count; i++) best = fmin_f(best, obstacle_clearance(world + 10 * i, p, time));
    return best;
}
// Group reductions by DPP lane swaps inside the group's own lanes (quad
// swaps 1 and 2, then the mirror of each 8-lane half row and of each 16-lane
// row): every step pairs a lane with one of the other half of its block, so
// after log2 G steps every lane of the group holds the combination of all G
// values.  A VALU operand modifier in place of an LDS-latency shuffle.
template <int STEP>
__device__ __forceinline__ uint32_t group_swap(uint32_t v) {
    constexpr int ctrl = STEP == 0 ? 0xB1 : STEP == 1 ? 0x4E : STEP == 2 ? 0x141 : 0x140;
    return uint32_t(__builtin_amdgcn_update_dpp(0, int(v), ctrl, 0xF, 0xF, false));
}
// min over the group of values that are never NaN and never -0 (then the
// minimum does not depend on the order of the pairings)
template <int G>
__device__ __forceinline__ float group_min(float v) {
    static_assert(G == 1 || G == 2 || G == 4 || G == 8 || G == 16, "DPP group within one row");
    if constexpr (G > 1) v = fmin_f(v, bits_float(group_swap<0>(float_bits(v))));
    if constexpr (G > 2) v = fmin_f(v, bits_float(group_swap<1>(float_bits(v))));
    if constexpr (G > 4) v = fmin_f(v, bits_float(group_swap<2>(float_bits(v))));
    if constexpr (G > 8) v = fmin_f(v, bits_float(group_swap<3>(float_bits(v))));
    return v;
}
template <int G>
__device__ __forceinline__ uint32_t group_or(uint32_t v) {
    static_assert(G == 1 || G == 2 || G == 4 || G == 8 || G == 16, "DPP group within one row");
    if constexpr (G > 1) v |= group_swap<0>(v);
    if constexpr (G > 2) v |= group_swap<1>(v);
    if constexpr (G > 4) v |= group_swap<2>(v);
    if constexpr (G > 8) v |= group_swap<3>(v);
    return v;
}

// The same clearance evaluated by a lane group: lane l takes obstacles l,
// l+G, ... and the group combines them (group_min).  For a finite point every
// term is finite and none is -0 (x - 0.18f rounds an exact cancellation to
// +0), so the minimum does not depend on the order and equals clearance_at.
// Call with the whole group active.
template <int G>
__device__ __forceinline__ float clearance_group(const float* world, uint32_t count, V p, float time, uint32_t lane) {
    float best = room_clearance(p);
    for (uint32_t i = lane; i < count; i += G) best = fmin_f(best, obstacle_clearance(world + 10 * i, p, time));
    if constexpr (G <= 16) return group_min<G>(best);
#pragma unroll
    for (int off = 1; off < G; off <<= 1) best = fmin_f(best, __shfl_xor(best, off, G));
    return best;
}

// clearance_group for a group whose env has at most G obstacles, all boxes
// (kind 0, fixed or at constant velocity): lane l holds obstacle l's record in
// registers (`o`, valid when `mine`), so no LDS read sits on the substep's
// dependency chain.  The same operations as room_clearance, obstacle_center
// and obstacle_clearance for a box, and the same order-free minimum.
// For a finite point no operand here is NaN, and no minimum or maximum sees a
// -0 whose sign could reach the result (the box terms are sums that cancel to
// +0 and every clearance ends in x - 0.18f), so the hardware min/max give
// fmin_f's and fmax_f's values.
template <int G>
__device__ __forceinline__ float clearance_boxes(const float (&o)[10], bool mine, V p, float time) {
    float best = __builtin_fminf(__builtin_fminf(p.x + 2, 14 - p.x),
                                 __builtin_fminf(__builtin_fminf(p.y + 5, 5 - p.y), __builtin_fminf(p.z, 5 - p.z))) -
                 0.18f;
    const V c = mk(o[1] + time * o[7], o[2] + time * o[8], o[3] + time * o[9]);
    const V q = sub3(p, c);
    const V k = mk(fabs_f(q.x) - o[4], fabs_f(q.y) - o[5], fabs_f(q.z) - o[6]);
    const float distance = len3(mk(__builtin_fmaxf(k.x, 0.0f), __builtin_fmaxf(k.y, 0.0f), __builtin_fmaxf(k.z, 0.0f))) +
                           __builtin_fminf(__builtin_fmaxf(k.x, __builtin_fmaxf(k.y, k.z)), 0.0f);
    const float oc = distance - 0.18f;
    best = mine ? __builtin_fminf(best, oc) : best;
    if constexpr (G > 1) best = __builtin_fminf(best, bits_float(group_swap<0>(float_bits(best))));
    if constexpr (G > 2) best = __builtin_fminf(best, bits_float(group_swap<1>(float_bits(best))));
    if constexpr (G > 4) best = __builtin_fminf(best, bits_float(group_swap<2>(float_bits(best))));
    if constexpr (G > 8) best = __builtin_fminf(best, bits_float(group_swap<3>(float_bits(best))));
    return best;
}

// sim.metal:43-48
__device__ __forceinline__ void rotation(const float q[4], float r[9]) {
    const float w = q[0], x = q[1], y = q[2], z = q[3];
    r[0] = 1 - 2 * (y * y + z * z); r[1] = 2 * (x * y - w * z); r[2] = 2 * (x * z + w * y);
    r[3] = 2 * (x * y + w * z); r[4] = 1 - 2 * (x * x + z * z); r[5] = 2 * (y * z - w * x);
    r[6] = 2 * (x * z - w * y); r[7] = 2 * (y * z + w * x); r[8] = 1 - 2 * (x * x + y * y);
}

// ---------------------------------------------------------------- plant
// x / b through the divisor's fp64 reciprocal R = RN64(1/b): the fp64 product
// x*R is within 2^-52 of x/b, closer than any fp32 rounding boundary that x/b
// is not on, so rounding it once to fp32 gives the correctly rounded x / b.
// Checked exhaustively on the GPU (all 2^32 numerators, signed zeros,
// subnormals, infinities and NaN) for the plant's divisors (rotor time
// constants, mass, 6) and fourteen others.  Three instructions in place of
// the eleven of a correctly rounded fp32 division.
__device__ __forceinline__ float div_r(float x, double R) { return (float)(double(x) * R); }

// ---------------------------------------------------------------- guidance
// Geometry-prior hint of a 184-input actor (guidance.hpp:38-98,
// nav_guidance), computed by one env's 8-lane group with one row of the 8x10
// pooled grid per lane.  The 3x3 nearest range and the 3x3 closing-speed
// risk around a cell are a min and a max over neighbours, so each is taken as
// a 3-row window through the neighbouring lanes (DPP row shifts) and then a
// 3-cell window along the lane's row; the risk contribution of a cell depends
// on that cell alone and is computed once.  The best cell and the
// goal cell are reduced over the group with the sequential scan's rule (the
// maximum; on equal values the first cell in row-major order), and the rest
// runs replicated in every lane.  `orow` is the env's observation row (pooled
// ranges / 12, current then previous), `cells` the 80 cell directions
// nav_ray(row, col) (computed on the host with the same fp32 operations),
// `inv_dt` = RN64(1 / max(sensor_dt, 1e-3)).
__device__ __forceinline__ float guid_atanh(float x) { return 0.5f * log_f((1.0f + x) / (1.0f - x)); }

// value of lane - 1 (UP) or lane + 1 (down) within a 16-lane DPP row; the
// caller masks the group's edge lanes
template <bool UP>
__device__ __forceinline__ float guid_row_shift(float x) {
    constexpr int ctrl = UP ? 0x111 : 0x101;  // row_shr:1 / row_shl:1
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), ctrl, 0xf, 0xf, true));
}

template <int G>
__device__ __forceinline__ void guidance_group(const float* orow, const float* __restrict__ cells, const float* goal_in,
                                               float goal_distance, const float* vel, float sensor_dt, double inv_dt,
                                               uint32_t lane, float (&hint)[3]) {
    static_assert(G == 8, "one pooled row per lane");
    const float gnorm = sqrt_f(goal_in[0] * goal_in[0] + goal_in[1] * goal_in[1] + goal_in[2] * goal_in[2]);
    if (gnorm < 1e-6f || goal_distance < 0.05f) {
        hint[0] = hint[1] = hint[2] = 0.0f;
        return;
    }
    const float goal[3] = {goal_in[0] / gnorm, goal_in[1] / gnorm, goal_in[2] / gnorm};
    const float speed = sqrt_f(vel[0] * vel[0] + vel[1] * vel[1] + vel[2] * vel[2]);
    const float stop_margin = 0.28f + speed * fmax_f(sensor_dt, 0.0f) + 0.25f * speed * speed;
    const bool temporal = sensor_dt > 1e-4f;
    const uint32_t row = lane;
    // this row's ranges and per-cell closing-speed risk (guidance.hpp:55-63: a
    // neighbour contributes min(0.2 u, 1) when its unexpected closing speed u
    // exceeds 0.5 m/s, else nothing; contributions are positive and the scan
    // starts from 0), then the 3-row windows through the neighbouring lanes
    float vn[10], vr[10];
#pragma unroll
    for (int j = 0; j < 10; j++) {
        const uint32_t k = row * 10 + j;
        const float now = orow[k] * 12.0f, old = orow[80 + k] * 12.0f;
        const float d0 = cells[3 * k], d1 = cells[3 * k + 1], d2 = cells[3 * k + 2];
        const float unexpected = div_r(old - now, inv_dt) - (vel[0] * d0 + vel[1] * d1 + vel[2] * d2);
        const bool hit = temporal & (old < 11.9f) & (now < 11.9f) & (unexpected > 0.5f);
        vn[j] = now;
        vr[j] = hit ? fmin_f(0.20f * unexpected, 1.0f) : 0.0f;
    }
    const bool has_up = row > 0, has_down = row < 7;
#pragma unroll
    for (int j = 0; j < 10; j++) {
        const float un = guid_row_shift<true>(vn[j]), dn = guid_row_shift<false>(vn[j]);
        const float ur = guid_row_shift<true>(vr[j]), dr = guid_row_shift<false>(vr[j]);
        vn[j] = has_up ? fmin_f(vn[j], un) : vn[j];
        vn[j] = has_down ? fmin_f(vn[j], dn) : vn[j];
        vr[j] = has_up ? fmax_f(vr[j], ur) : vr[j];
        vr[j] = has_down ? fmax_f(vr[j], dr) : vr[j];
    }
    // 3-cell windows along the row; the row's cells scored in order
    float bscore = -1e20f, brange = 0.0f, galign = -1e20f, gnear = 0.0f, near0 = 0.0f;
    uint32_t bcell = 80, gcell = 80;  // 80: none (the scan's initial state)
#pragma unroll
    for (int j = 0; j < 10; j++) {
        float nearby = fmin_f(12.0f, vn[j]), r = vr[j];
        if (j > 0) { nearby = fmin_f(nearby, vn[j - 1]); r = fmax_f(r, vr[j - 1]); }
        if (j < 9) { nearby = fmin_f(nearby, vn[j + 1]); r = fmax_f(r, vr[j + 1]); }
        if (j == 0) near0 = nearby;
        const uint32_t c = row * 10 + j;
        const float alignment = cells[3 * c] * goal[0] + cells[3 * c + 1] * goal[1] + cells[3 * c + 2] * goal[2];
        const float safe_range = fmax_f(nearby - r, 0.0f);
        const float score = 1.4f * alignment + 0.12f * fmin_f(safe_range, 6.0f);
        if (score > bscore) { bscore = score; bcell = c; brange = safe_range; }
        if (alignment > galign) { galign = alignment; gcell = c; gnear = nearby; }
    }
#pragma unroll
    for (int off = 1; off < G; off <<= 1) {
        const float os = __shfl_xor(bscore, off, G), orr = __shfl_xor(brange, off, G);
        const uint32_t oc = __shfl_xor(bcell, off, G);
        if (os > bscore || (os == bscore && oc < bcell)) { bscore = os; bcell = oc; brange = orr; }
        const float oa = __shfl_xor(galign, off, G), on = __shfl_xor(gnear, off, G);
        const uint32_t og = __shfl_xor(gcell, off, G);
        if (oa > galign || (oa == galign && og < gcell)) { galign = oa; gcell = og; gnear = on; }
    }
    // no goal cell (non-finite alignments only): the scan's fallback is cell 0
    const float near_cell0 = __shfl(near0, 0, G);
    float best_dir[3] = {1.0f, 0.0f, 0.0f};
    if (bcell < 80) { best_dir[0] = cells[3 * bcell]; best_dir[1] = cells[3 * bcell + 1]; best_dir[2] = cells[3 * bcell + 2]; }
    const float max_speed = 1.6f;
    const float desired_speed = fmin_f(max_speed, sqrt_f(4.0f * fmax_f(goal_distance - 0.28f, 0.0f)));
    const float direct_range = fmax_f(gcell < 80 ? gnear : near_cell0, 0.0f);
    float direction[3] = {best_dir[0], best_dir[1], best_dir[2]}, available = brange;
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
#pragma unroll
        for (int i = 0; i < 3; i++) direction[i] /= fmax_f(norm, 1e-6f);
    }
#pragma unroll
    for (int i = 0; i < 3; i++) hint[i] = guid_atanh(fraction * direction[i]);
}


// Pooled cells of the top two grid rows farther than 2.5 m (sim.metal:233, 236).
__device__ __forceinline__ float overhead_cells(const float* o) {
    float overhead = 0.0f;
#pragma unroll
    for (int k = 0; k < 20; k++) overhead += o[k] * 12.0f > 2.5f ? 1.0f : 0.0f;
    return overhead;
}
// sim.metal:233: evaluation modes 9-21 of the 184-input actor pull the means
// toward the hint (inputs 181-183) by a mode-dependent scale.
__device__ __forceinline__ void guided_mode_means(uint32_t mode, const float* o, float (&mean)[4]) {
    float scale = (mode == 9 || mode == 13) ? 0.0f
                  : ((mode == 10 || mode == 14 || mode == 16) ? 0.25f : (mode == 15 ? 1.0f : 0.5f));
    if (mode >= 17) scale = 0.25f + 0.75f * (overhead_cells(o) / 20.0f);
    if (mode == 12) {
        float near = 12.0f;
        for (int k = 0; k < 80; k++) near = fmin_f(near, o[k] * 12.0f);
        scale = clamp_f((near - .3f) / 2, 0.2f, 1.0f);
    }
#pragma unroll
    for (int j = 0; j < 3; j++) {
        const float prior = o[MDN_ACTOR_OBS_PRIOR - 3 + j];
        mean[j] = prior + scale * (mean[j] - prior);
    }
    mean[3] *= scale;
    if (mode == 16) {
        const float yaw = atan2_f(o[161], o[160]);
        mean[3] += guid_atanh(clamp_f(yaw * 1.5f, -.85f, .85f));
    }
}

// fp64 reciprocals of the plant's constant divisors
struct PhysRecip {
    double mass, rise[4], fall[4];
};
// The Crazyflie profile's reciprocals, RN64(1/x) as phys_recip forms them.
constexpr PhysRecip kCrazyflieRecip = {
    1.0 / double(mdn::kCrazyflie.mass),
    {1.0 / double(mdn::kCrazyflie.rotor_time_constants_rising[0]), 1.0 / double(mdn::kCrazyflie.rotor_time_constants_rising[1]),
     1.0 / double(mdn::kCrazyflie.rotor_time_constants_rising[2]), 1.0 / double(mdn::kCrazyflie.rotor_time_constants_rising[3])},
    {1.0 / double(mdn::kCrazyflie.rotor_time_constants_falling[0]), 1.0 / double(mdn::kCrazyflie.rotor_time_constants_falling[1]),
     1.0 / double(mdn::kCrazyflie.rotor_time_constants_falling[2]), 1.0 / double(mdn::kCrazyflie.rotor_time_constants_falling[3])}};
// The plant a kernel instance reads: its LDS copy of the launch's plant, or
// (CF) the Crazyflie profile as compile-time constants, which the compiler
// folds into the physics instructions as immediates.
template <bool CF>
__device__ __forceinline__ const MdnPhysicsParams& plant_ref(const MdnPhysicsParams& lds) {
    if constexpr (CF) return mdn::kCrazyflie; else return lds;
}
__device__ __forceinline__ PhysRecip phys_recip(const MdnPhysicsParams& P) {
    PhysRecip r;
    r.mass = 1.0 / double(P.mass);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        r.rise[i] = 1.0 / double(P.rotor_time_constants_rising[i]);
        r.fall[i] = 1.0 / double(P.rotor_time_constants_falling[i]);
    }
    return r;
}

// physics.hpp:60-112
__device__ __forceinline__ void derivative(const MdnPhysicsParams& P, const PhysRecip& RP, const State& s,
                                           const float sp[4], const float wind[3], State& d) {
    float thrust[3] = {0, 0, 0}, torque[3] = {0, 0, 0};
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float speed = s.rpm[r];
        const float* c = &P.rotor_thrust_coefficients[3 * r];
        const float magnitude = c[0] + c[1] * speed + c[2] * speed * speed;
        float rt[3];
        const float* dir = &P.rotor_thrust_directions[3 * r];
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            rt[i] = dir[i] * magnitude;
            thrust[i] += rt[i];
            torque[i] += P.rotor_torque_directions[3 * r + i] * magnitude * P.rotor_torque_constants[r];
        }
        const float* a = &P.rotor_positions[3 * r];
        const float arm0 = a[1] * rt[2] - a[2] * rt[1];
        const float arm1 = a[2] * rt[0] - a[0] * rt[2];
        const float arm2 = a[0] * rt[1] - a[1] * rt[0];
        torque[0] += arm0; torque[1] += arm1; torque[2] += arm2;
    }
#pragma unroll
    for (int i = 0; i < 3; ++i) d.p[i] = s.v[i];
    const float* q = s.q;
    const float* w = s.w;
    d.q[0] = -q[1] * w[0] - q[2] * w[1] - q[3] * w[2];
    d.q[1] = q[0] * w[0] + q[2] * w[2] - q[3] * w[1];
    d.q[2] = q[0] * w[1] + q[3] * w[0] - q[1] * w[2];
    d.q[3] = q[0] * w[2] + q[1] * w[1] - q[2] * w[0];
#pragma unroll
    for (int i = 0; i < 4; ++i) d.q[i] *= 0.5f;
    // rotate_body_to_world (physics.hpp:51-58)
    const float tx = 2.0f * (q[2] * thrust[2] - q[3] * thrust[1]);
    const float ty = 2.0f * (q[3] * thrust[0] - q[1] * thrust[2]);
    const float tz = 2.0f * (q[1] * thrust[1] - q[2] * thrust[0]);
    d.v[0] = thrust[0] + q[0] * tx + q[2] * tz - q[3] * ty;
    d.v[1] = thrust[1] + q[0] * ty + q[3] * tx - q[1] * tz;
    d.v[2] = thrust[2] + q[0] * tz + q[1] * ty - q[2] * tx;
#pragma unroll
    for (int i = 0; i < 3; ++i) d.v[i] = div_r(d.v[i], RP.mass) + P.gravity_world[i] + div_r(wind[i], RP.mass);
    float am[3] = {0, 0, 0};
#pragma unroll
    for (int row = 0; row < 3; ++row)
#pragma unroll
        for (int col = 0; col < 3; ++col) am[row] += P.inertia[3 * row + col] * w[col];
    const float g0 = w[1] * am[2] - w[2] * am[1];
    const float g1 = w[2] * am[0] - w[0] * am[2];
    const float g2 = w[0] * am[1] - w[1] * am[0];
    am[0] = torque[0] - g0; am[1] = torque[1] - g1; am[2] = torque[2] - g2;
#pragma unroll
    for (int row = 0; row < 3; ++row) {
        d.w[row] = 0.0f;
#pragma unroll
        for (int col = 0; col < 3; ++col) d.w[row] += P.inertia_inverse[3 * row + col] * am[col];
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const double inv_tau = sp[r] >= s.rpm[r] ? RP.rise[r] : RP.fall[r];
        d.rpm[r] = div_r(sp[r] - s.rpm[r], inv_tau);
    }
}

// derivative() for a plant of the standard quadrotor structure (the host
// checks it per launch): every rotor thrusts along body z (direction
// (0, 0, 1)) with a torque direction (0, 0, +-1), rotors sit in the z = 0
// plane, the inertia and its inverse are diagonal and gravity points along
// z.  The terms that structure makes zero are left out; every other term is
// the same operation on the same operands in the same order, so each
// derivative value equals derivative()'s (x + 0 = x and 0 - y = -y exactly;
// only the sign of a zero may differ, and the derivative has no operation -
// a division by a computed value, a sign test - that turns the sign of a zero
// into a difference of value).  Those values reach the state only as addends
// of state components, so when no state component is -0 (no_negative_zero)
// every stage state and the next state are bit-identical: s + (+-0) is s for
// s != 0 and +0 for s = +0.  wm = wind / mass, formed once per tick with the
// same division.
__device__ __forceinline__ void derivative_quad(const MdnPhysicsParams& P, const PhysRecip& RP, const State& s,
                                                const float sp[4], const float wm[3], State& d) {
    float m[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float speed = s.rpm[r];
        const float* c = &P.rotor_thrust_coefficients[3 * r];
        m[r] = c[0] + c[1] * speed + c[2] * speed * speed;
    }
    const float* a = P.rotor_positions;
    const float* td = P.rotor_torque_directions;
    const float* K = P.rotor_torque_constants;
    // thrust (0, 0, T); torque from the rotor arms (y m, -x m, 0) and the
    // rotor drag (0, 0, td m K), accumulated rotor by rotor as physics.hpp:70-86
    const float T = ((m[0] + m[1]) + m[2]) + m[3];
    const float t0 = ((a[1] * m[0] + a[4] * m[1]) + a[7] * m[2]) + a[10] * m[3];
    const float t1 = ((-(a[0] * m[0]) - a[3] * m[1]) - a[6] * m[2]) - a[9] * m[3];
    const float t2 = ((td[2] * m[0] * K[0] + td[5] * m[1] * K[1]) + td[8] * m[2] * K[2]) + td[11] * m[3] * K[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) d.p[i] = s.v[i];
    const float* q = s.q;
    const float* w = s.w;
    d.q[0] = -q[1] * w[0] - q[2] * w[1] - q[3] * w[2];
    d.q[1] = q[0] * w[0] + q[2] * w[2] - q[3] * w[1];
    d.q[2] = q[0] * w[1] + q[3] * w[0] - q[1] * w[2];
    d.q[3] = q[0] * w[2] + q[1] * w[1] - q[2] * w[0];
#pragma unroll
    for (int i = 0; i < 4; ++i) d.q[i] *= 0.5f;
    // rotate_body_to_world (physics.hpp:51-58) of (0, 0, T)
    const float tx = 2.0f * (q[2] * T);
    const float ty = 2.0f * -(q[1] * T);
    d.v[0] = q[0] * tx - q[3] * ty;
    d.v[1] = q[0] * ty + q[3] * tx;
    d.v[2] = T + q[1] * ty - q[2] * tx;
    d.v[0] = div_r(d.v[0], RP.mass) + wm[0];
    d.v[1] = div_r(d.v[1], RP.mass) + wm[1];
    d.v[2] = div_r(d.v[2], RP.mass) + P.gravity_world[2] + wm[2];
    const float am0 = P.inertia[0] * w[0], am1 = P.inertia[4] * w[1], am2 = P.inertia[8] * w[2];
    const float g0 = w[1] * am2 - w[2] * am1;
    const float g1 = w[2] * am0 - w[0] * am2;
    const float g2 = w[0] * am1 - w[1] * am0;
    d.w[0] = P.inertia_inverse[0] * (t0 - g0);
    d.w[1] = P.inertia_inverse[4] * (t1 - g1);
    d.w[2] = P.inertia_inverse[8] * (t2 - g2);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const double inv_tau = sp[r] >= s.rpm[r] ? RP.rise[r] : RP.fall[r];
        d.rpm[r] = div_r(sp[r] - s.rpm[r], inv_tau);
    }
}

// true when no component of s is -0 (the condition derivative_quad needs;
// a physics step keeps it, since a sum is -0 only when both addends are)
__device__ __forceinline__ bool no_negative_zero(const State& s) {
    const float* a = &s.p[0];
    bool ok = true;
#pragma unroll
    for (int i = 0; i < 17; ++i) ok = ok && float_bits(a[i]) != 0x80000000u;
    return ok;
}

__device__ __forceinline__ void axpy_state(const State& s, const State& d, float scale, State& out) {
    const float* a = &s.p[0];
    const float* b = &d.p[0];
    float* o = &out.p[0];
#pragma unroll
    for (int i = 0; i < 17; ++i) o[i] = a[i] + scale * b[i];
}

// physics.hpp:122-179.  QUAD: the standard-structure derivative
// (derivative_quad; `wind` is then wind / mass).
template <bool QUAD = false>
__device__ __forceinline__ void physics_step(const MdnPhysicsParams& P, const PhysRecip& RP, const State& s,
                                             const float action[4], const float wind[3], State& next) {
    float sp[4];
    const float half = (P.action_max - P.action_min) * 0.5f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        // the clamps to nonzero bounds as a median of three: for a non-NaN
        // value it is the comparisons' result, -0 included (a NaN state is
        // rejected by the caller's validity check either way)
        const float a = __builtin_amdgcn_fmed3f(action[i], -1.0f, 1.0f);
        sp[i] = a * half + P.action_min + half;
    }
    // k1 + 2 k2 + 2 k3 + k4 accumulated left to right as it is written in
    // physics.hpp:133-142, so only one stage derivative is live at a time.
    State k, acc, tmp;
    if constexpr (QUAD) derivative_quad(P, RP, s, sp, wind, k); else derivative(P, RP, s, sp, wind, k);
    axpy_state(s, k, 0.5f * P.dt, tmp);
    acc = k;
    if constexpr (QUAD) derivative_quad(P, RP, tmp, sp, wind, k); else derivative(P, RP, tmp, sp, wind, k);
    axpy_state(s, k, 0.5f * P.dt, tmp);
    {
        float* a = &acc.p[0];
        const float* b = &k.p[0];
#pragma unroll
        for (int i = 0; i < 17; ++i) a[i] = fma_f(2.0f, b[i], a[i]);  // = a + 2b: 2b is exact
    }
    if constexpr (QUAD) derivative_quad(P, RP, tmp, sp, wind, k); else derivative(P, RP, tmp, sp, wind, k);
    axpy_state(s, k, P.dt, tmp);
    {
        float* a = &acc.p[0];
        const float* b = &k.p[0];
#pragma unroll
        for (int i = 0; i < 17; ++i) a[i] = fma_f(2.0f, b[i], a[i]);  // = a + 2b: 2b is exact
    }
    if constexpr (QUAD) derivative_quad(P, RP, tmp, sp, wind, k); else derivative(P, RP, tmp, sp, wind, k);
    const float* a0 = &s.p[0];
    const float* ak = &k.p[0];
    float* ac = &acc.p[0];
    float* o = &next.p[0];
#pragma unroll
    for (int i = 0; i < 17; ++i) o[i] = a0[i] + div_r(P.dt * (ac[i] + ak[i]), 1.0 / 6.0);
    const float norm = sqrt_f(next.q[0] * next.q[0] + next.q[1] * next.q[1] + next.q[2] * next.q[2] + next.q[3] * next.q[3]);
    const double inv_norm = 1.0 / double(norm);
#pragma unroll
    for (int i = 0; i < 4; ++i) next.q[i] = div_r(next.q[i], inv_norm);
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        next.p[i] = __builtin_amdgcn_fmed3f(next.p[i], -P.position_limit, P.position_limit);
        next.v[i] = __builtin_amdgcn_fmed3f(next.v[i], -P.velocity_limit, P.velocity_limit);
        next.w[i] = __builtin_amdgcn_fmed3f(next.w[i], -P.angular_velocity_limit, P.angular_velocity_limit);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (next.rpm[i] < P.action_min) next.rpm[i] = P.action_min;
        if (next.rpm[i] > P.action_max) next.rpm[i] = P.action_max;
    }
}

// ---------------------------------------------------------------- world generation
// world.hpp:104-318, written over a WWorld word array; multi-draw argument
// lists are sequenced left to right.
struct WorldGen {
    float* w;  // WORLD_WORDS words
    __device__ uint32_t count() const { return float_bits(w[160]); }
    __device__ void set_count(uint32_t c) { w[160] = bits_float(c); }
    __device__ float goal(int j) const { return w[163 + j]; }
    __device__ void add(uint32_t kind, V c, V e, V v) {
        const uint32_t n = count();
        if (n >= 16) return;
        float* o = w + 10 * n;
        o[0] = bits_float(kind);
        o[1] = c.x; o[2] = c.y; o[3] = c.z;
        o[4] = e.x; o[5] = e.y; o[6] = e.z;
        o[7] = v.x; o[8] = v.y; o[9] = v.z;
        set_count(n + 1);
    }
    __device__ void box(V c, V e) { add(0, c, e, mk(0, 0, 0)); }
    __device__ void table(float x, float y, float hx, float hy, float top) {
        const float slab = 0.08f, underside = top - slab;
        box(mk(x, y, top), mk(hx, hy, slab));
        const float lx = hx - 0.12f, ly = hy - 0.12f, leg = 0.08f;
        const float lcz = underside * 0.5f, lhz = underside * 0.5f;
        box(mk(x - lx, y - ly, lcz), mk(leg, leg, lhz));
        box(mk(x - lx, y + ly, lcz), mk(leg, leg, lhz));
        box(mk(x + lx, y - ly, lcz), mk(leg, leg, lhz));
        box(mk(x + lx, y + ly, lcz), mk(leg, leg, lhz));
    }
    __device__ float route_y(float x, float distance) const { return goal(1) * (x / distance); }
    __device__ void doorway(float wall_x, float gy, float gz, float hg, float hgz) {
        const float low_y = gy - hg, high_y = gy + hg, low_z = gz - hgz, high_z = gz + hgz, whx = 0.12f;
        box(mk(wall_x, (-5.0f + low_y) * 0.5f, 2.5f), mk(whx, (low_y + 5.0f) * 0.5f, 2.5f));
        box(mk(wall_x, (high_y + 5.0f) * 0.5f, 2.5f), mk(whx, (5.0f - high_y) * 0.5f, 2.5f));
        box(mk(wall_x, 0, low_z * 0.5f), mk(whx, 5.0f, low_z * 0.5f));
        box(mk(wall_x, 0, (high_z + 5.0f) * 0.5f), mk(whx, 5.0f, (5.0f - high_z) * 0.5f));
    }
    __device__ void goal_span(uint32_t& rng, float distance) {
        const float span = fmin_f(fmax_f(distance, 3.0f), 10.0f);
        w[163] = span * (0.90f + 0.10f * ur(rng));
        w[164] = (ur(rng) - 0.5f) * 1.20f;
        w[165] = 1.10f + 0.80f * ur(rng);
    }
    // Four bounded movers (kind 3, world.hpp:26-41: size = {radius, travel
    // amplitude, phase}, velocity = direction times peak speed): radius
    // U[0.2, 0.5] m, peak speed U[0.3, 1.5] m/s along a horizontal heading,
    // amplitude U[0.5, 2] m, phase U[-pi, pi), centres spread along the route
    // to `reach`.  Every draw is a statement of its own (draw order fixed).
    __device__ void movers(uint32_t& rng, float reach) {
        for (int i = 0; i < 4; i++) {
            const float cx = 1.5f + ur(rng) * fmax_f(0.5f, reach - 2.5f);
            const float cy = (ur(rng) - 0.5f) * 5.0f;
            const float cz = 0.8f + ur(rng) * 1.6f;
            const float radius = 0.2f + 0.3f * ur(rng);
            const float speed = 0.3f + 1.2f * ur(rng);
            const float heading = 6.28318530718f * ur(rng);
            const float amplitude = 0.5f + 1.5f * ur(rng);
            const float phase = (ur(rng) - 0.5f) * 6.28318530718f;
            float sh, ch;
            sincos_f(heading, &sh, &ch);
            add(3, mk(cx, cy, cz), mk(radius, amplitude, phase), mk(speed * ch, speed * sh, 0.0f));
        }
    }
    // The combined course of navigation_challenge_tasks.py:47-117 (kind
    // "combined") with xorshift draws: a 3.2 m corridor with a side opening
    // at 0.59 L, staggered openings at 0.32 L and 0.68 L, a hanging beam at
    // 0.5 L and one bounded sphere crossing the side opening; the start
    // height is the reset's 1.5 m.  Ten obstacles.
    __device__ void course(uint32_t& rng) {
        const float length = 8.5f + 3.0f * ur(rng);
        const float yg = (ur(rng) - 0.5f) * 0.4f;
        const float z = 1.5f, width = 3.2f, cross = length * 0.59f;
        w[163] = length; w[164] = yg; w[165] = z;
        for (int side = -1; side <= 1; side += 2) {
            const float y = float(side) * (width * 0.5f + 0.06f);
            const float l0 = -2.0f, h0 = cross - 0.7f, l1 = cross + 0.7f, h1 = 14.0f;
            box(mk((l0 + h0) * 0.5f, y, 2.5f), mk((h0 - l0) * 0.5f, 0.06f, 2.5f));
            box(mk((l1 + h1) * 0.5f, y, 2.5f), mk((h1 - l1) * 0.5f, 0.06f, 2.5f));
        }
        const bool hard = ur(rng) < 0.5f;
        const float ug = ur(rng);
        const float gap = hard ? 0.85f + 0.35f * ug : 1.15f + 0.40f * ug;
        const float uo = ur(rng);
        const float offset = hard ? 0.65f + 0.20f * uo : 0.45f + 0.20f * uo;
        const float sign = ur(rng) < 0.5f ? -1.0f : 1.0f;
        for (int stage = 0; stage < 2; stage++) {
            const float x = length * (stage == 0 ? 0.32f : 0.68f);
            const float cy = sign * offset * (stage == 0 ? 1.0f : -1.0f);
            const float l0 = -width * 0.5f, h0 = cy - gap * 0.5f, l1 = cy + gap * 0.5f, h1 = width * 0.5f;
            box(mk(x, (l0 + h0) * 0.5f, 2.5f), mk(0.12f, (h0 - l0) * 0.5f, 2.5f));
            box(mk(x, (l1 + h1) * 0.5f, 2.5f), mk(0.12f, (h1 - l1) * 0.5f, 2.5f));
        }
        box(mk(length * 0.5f, 0.0f, 3.35f), mk(0.25f, width * 0.5f, 1.65f));
        const float us = ur(rng);
        const float speed = hard ? 0.65f + 0.35f * us : 0.35f + 0.30f * us;
        const float phase = -1.57079632679f + (ur(rng) - 0.5f) * 0.5f;
        const float dir = ur(rng) < 0.5f ? -1.0f : 1.0f;
        const float amplitude = 2.2f + 1.2f * ur(rng);
        add(3, mk(cross, 0.0f, z), mk(0.28f, amplitude, phase), mk(0.0f, dir * speed, 0.0f));
    }
    // Like wgenerate, slots beyond the new count keep their previous contents.
    __device__ void generate(uint32_t seed, uint32_t family, float distance) {
        uint32_t rng = seed ? seed : 1;
        w[161] = bits_float(seed);
        w[162] = bits_float(family);
        set_count(family == 0 ? 0 : 8);
        w[163] = distance;
        w[164] = (ur(rng) - 0.5f) * 2;
        w[165] = 1.5f + (ur(rng) - 0.5f) * 0.8f;
        if (family == 4) {  // world.hpp:138-147
            set_count(0);
            const float wall_x = distance * (0.42f + 0.16f * ur(rng));
            const float rf = wall_x / distance;
            const float gy = goal(1) * rf + (ur(rng) - 0.5f) * 1.20f;
            const float hg = 0.40f + 0.30f * ur(rng);
            const float rz = 1.5f + (goal(2) - 1.5f) * rf;
            const float gz = rz + (ur(rng) - 0.5f) * 0.20f;
            const float hgz = 0.65f + 0.25f * ur(rng);
            doorway(wall_x, gy, gz, hg, hgz);
            return;
        }
        if (family == 5) {  // world.hpp:161-176
            set_count(0);
            const float x = distance * (0.45f + 0.10f * ur(rng));
            const float y = route_y(x, distance) + (ur(rng) - 0.5f) * 0.20f;
            if (ur(rng) < 0.5f) {
                const float hx = 0.55f + 0.20f * ur(rng);
                const float hy = 0.75f + 0.20f * ur(rng);
                const float top = 1.55f + 0.50f * ur(rng);
                table(x, y, hx, hy, top);
            } else {
                const float hx = 0.60f + 0.20f * ur(rng);
                const float hy = 0.80f + 0.20f * ur(rng);
                const float height = 1.35f + 0.80f * ur(rng);
                box(mk(x, y, height * 0.5f), mk(hx, hy, height * 0.5f));
            }
            return;
        }
        if (family == 6) {  // world.hpp:177-201
            set_count(0);
            const float table_x = distance * (0.46f + 0.08f * ur(rng));
            const float table_y = route_y(table_x, distance) + (ur(rng) - 0.5f) * 0.16f;
            const float thx = 0.58f + 0.10f * ur(rng);
            const float thy = 0.76f + 0.10f * ur(rng);
            const float ttop = 1.62f + 0.42f * ur(rng);
            table(table_x, table_y, thx, thy, ttop);
            const float counter_x = distance * 0.22f;
            const float counter_y = route_y(counter_x, distance) - 1.30f;
            const float counter_h = 1.55f + 0.45f * ur(rng);
            box(mk(counter_x, counter_y, counter_h * 0.5f), mk(0.30f, 0.50f, counter_h * 0.5f));
            const float sphere_x = distance * 0.72f;
            const float sphere_y = route_y(sphere_x, distance) + 1.35f;
            const float sphere_r = 0.34f + 0.10f * ur(rng);
            const float sphere_z = 1.05f + 1.10f * ur(rng);
            const float sign = ur(rng) < 0.5f ? -1.0f : 1.0f;
            const float sphere_vy = sign * (0.18f + 0.16f * ur(rng));
            add(1, mk(sphere_x, sphere_y, sphere_z), mk(sphere_r, sphere_r, sphere_r), mk(0, sphere_vy, 0));
            const float pole_r0 = 0.20f + 0.08f * ur(rng);
            const float pole_r1 = 0.20f + 0.08f * ur(rng);
            add(2, mk(distance * 0.34f, route_y(distance * 0.34f, distance) + 2.05f, 2.5f), mk(pole_r0, pole_r0, 2.5f), mk(0, 0, 0));
            add(2, mk(distance * 0.82f, route_y(distance * 0.82f, distance) - 2.05f, 2.5f), mk(pole_r1, pole_r1, 2.5f), mk(0, 0, 0));
            const float low_box_x = distance * 0.74f;
            const float low_box_y = route_y(low_box_x, distance) - 0.88f;
            box(mk(low_box_x, low_box_y, 0.48f), mk(0.34f, 0.30f, 0.48f));
            return;
        }
        if (family == 8) {  // world.hpp:148-160
            set_count(0);
            for (uint32_t door = 0; door < 2; door++) {
                const float u0 = ur(rng);
                const float fraction = door == 0 ? 0.33f + 0.02f * (u0 - 0.5f) : 0.67f + 0.02f * (u0 - 0.5f);
                const float wall_x = distance * fraction;
                const float rf = wall_x / distance;
                const float gy = route_y(wall_x, distance) + (ur(rng) - 0.5f) * 1.00f;
                const float rz = 1.5f + (goal(2) - 1.5f) * rf;
                const float gz = rz + (ur(rng) - 0.5f) * 0.24f;
                const float hg = 0.40f + 0.30f * ur(rng);
                const float hgz = 0.65f + 0.25f * ur(rng);
                doorway(wall_x, gy, gz, hg, hgz);
            }
            return;
        }
        if (family == 10 || family == 11) {  // world.hpp:202-222
            set_count(0);
            const float drone_speed = 1.5f;
            uint32_t tr = seed ^ 0x9e3779b9u;
            if (tr == 0) tr = 1;
            const float lateral = (ur(tr) - 0.5f) * 0.20f;
            const float vertical = (ur(tr) - 0.5f) * 0.16f;
            const uint32_t speed_choice = xs(tr) % 3;
            const float threat_speed = speed_choice == 0 ? 0.5f : (speed_choice == 1 ? 1.0f : 2.0f);
            const float nominal_ttc = 0.7f + 0.8f * ur(tr);
            const float combined_radius = 0.18f + 0.35f;
            V center, velocity = mk(0, 0, 0);
            if (family == 10) {
                center = mk((drone_speed + threat_speed) * nominal_ttc + combined_radius, lateral, 1.5f + vertical);
                velocity.x = -threat_speed;
            } else {
                center = mk(drone_speed * nominal_ttc, -threat_speed * nominal_ttc + lateral, 1.5f + vertical);
                velocity.y = threat_speed;
            }
            w[163] = 4.0f; w[164] = 0.0f; w[165] = 1.5f;
            add(1, center, mk(0.35f, 0.35f, 0.35f), velocity);
            return;
        }
        if (family == 14) {  // world.hpp:226-241
            set_count(0);
            const float difficulty = ur(rng);
            goal_span(rng, distance);
            const float wall_x = goal(0) * (0.24f + 0.04f * ur(rng));
            const float gap_x = goal(0) * (0.70f + 0.08f * difficulty);
            const float lane_width = 1.80f - 0.80f * difficulty;
            const float lane_edge = 5.0f - lane_width;
            const float wall_y = (-5.0f + lane_edge) * 0.5f;
            const float wall_half_y = (lane_edge + 5.0f) * 0.5f;
            box(mk(wall_x, wall_y, 2.5f), mk(0.15f, wall_half_y, 2.5f));
            box(mk((wall_x + gap_x) * 0.5f, lane_edge + 0.03f, 2.5f), mk((gap_x - wall_x) * 0.5f + 0.15f, 0.15f, 2.5f));
            return;
        }
        if (family == 15) {  // world.hpp:242-269
            set_count(0);
            const float difficulty = ur(rng);
            goal_span(rng, distance);
            const float wall_1 = goal(0) * (0.16f + 0.02f * ur(rng));
            const float wall_2 = goal(0) * 0.85f;
            const float gap_1 = -(0.60f + 0.80f * difficulty);
            const float gap_2 = +(0.60f + 0.80f * difficulty);
            const float gap_half = 0.85f - 0.30f * difficulty;
            const float gap_half_z = 0.85f - 0.10f * difficulty;
            doorway(wall_1, gap_1, 1.50f, gap_half, gap_half_z);
            doorway(wall_2, gap_2, 1.50f, gap_half, gap_half_z);
            const float table_x = goal(0) * 0.50f;
            const float table_y = (ur(rng) - 0.5f) * 0.20f;
            const float table_half_x = fmin_f(0.45f, goal(0) * 0.06f);
            const float table_half_y = 0.60f + 0.20f * difficulty;
            const float table_top = 1.45f + 0.25f * difficulty;
            table(table_x, table_y, table_half_x, table_half_y, table_top);
            box(mk(goal(0) * 0.38f, 3.75f, 0.55f), mk(0.22f, 0.35f, 0.55f));
            box(mk(goal(0) * 0.50f, -3.80f, 0.80f), mk(0.25f, 0.35f, 0.80f));
            box(mk(goal(0) * 0.62f, 3.70f, 0.50f), mk(0.22f, 0.40f, 0.50f));
            return;
        }
        if (family == 16) {  // world.hpp:270-291
            set_count(0);
            const float difficulty = ur(rng);
            goal_span(rng, distance);
            const float low_x = goal(0) * (0.14f + 0.02f * (1.0f - difficulty));
            const float overhead_x = goal(0) * (0.46f + 0.02f * difficulty);
            const float choice_x = goal(0) * (0.76f + 0.02f * difficulty);
            const float low_top = 1.50f + 0.25f * difficulty;
            const float overhead_bottom = 2.80f - 0.20f * difficulty;
            const float choice_half_z = 0.10f + 0.05f * difficulty;
            box(mk(low_x, 0, low_top * 0.5f), mk(0.12f, 5.0f, low_top * 0.5f));
            const float overhead_half_z = (5.0f - overhead_bottom) * 0.5f;
            box(mk(overhead_x, 0, overhead_bottom + overhead_half_z), mk(0.12f, 5.0f, overhead_half_z));
            box(mk(choice_x, 0, 2.0f + choice_half_z), mk(0.10f, 5.0f, choice_half_z));
            return;
        }
        if (family == MDN_FAMILY_COURSE) {
            set_count(0);
            course(rng);
            return;
        }
        const bool mover_world = family == MDN_FAMILY_MOVERS || family == MDN_FAMILY_MOVERS_LONG;
        float reach = distance;
        if (family == MDN_FAMILY_MOVERS_LONG) {  // a long goal, 8-13 m (the room ends at x = 14)
            reach = 8.0f + 5.0f * ur(rng);
            w[163] = reach;
        }
        // world.hpp:311-317: sixteen random slots, the first eight live
        for (uint32_t i = 0; i < 16; i++) {
            float* o = w + 10 * i;
            o[0] = bits_float(family == 2 ? 2u : (family == 3 ? 1u : 0u));
            o[1] = 1.2f + ur(rng) * fmax_f(0.1f, reach - 2.2f);
            o[2] = (ur(rng) - 0.5f) * 7;
            o[3] = family == 2 ? 2.5f : 0.6f + ur(rng) * 3;
            o[4] = 0.2f + ur(rng) * 0.35f;
            o[5] = 0.3f + ur(rng) * 0.55f;
            o[6] = family == 2 ? 2.5f : 0.2f + ur(rng) * 0.75f;
            o[7] = 0;
            o[8] = family == 3 ? (ur(rng) - 0.5f) * 0.8f : 0;
            o[9] = 0;
        }
        if (mover_world) movers(rng, reach);  // slots 8-11
    }
};

// world.hpp:293-298
__device__ __forceinline__ uint32_t training_family(uint32_t family, uint32_t& rng) {
    if (family == 7) return xs(rng) % 7;
    if (family == 9 || family == 12) {
        const uint32_t choice = xs(rng) % 4;
        return choice < 2 ? 4 : (choice == 2 ? 5 : xs(rng) % 7);
    }
    if (family == 13) {
        const uint32_t choice = xs(rng) % 6;
        if (choice < 2) return 4;
        if (choice == 2) return 5;
        if (choice == 3) return xs(rng) % 7;
        return choice == 4 ? 10 : 11;
    }
    return family;
}

}  // namespace nav
