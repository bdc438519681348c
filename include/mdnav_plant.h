/*
 * mdnav_plant.h — the L2F Crazyflie plant (physics.hpp:184-219) as a
 * constant expression, shared by the host (mdn::crazyflie_params) and the
 * device.  The device builds rollout instances in which every plant constant
 * is this profile folded into the instructions as an immediate operand; the
 * host selects them only when the simulator's plant equals the profile byte
 * for byte, so both instances compute the same bits.
 */
#ifndef MDNAV_PLANT_H
#define MDNAV_PLANT_H

#include "mdnav_types.h"

namespace mdn {

constexpr MdnPhysicsParams crazyflie_profile() {
    MdnPhysicsParams p{};
    const float positions[12] = {.028f, -.028f, 0, -.028f, -.028f, 0, -.028f, .028f, 0, .028f, .028f, 0};
    const float torque_z[4] = {-1, 1, -1, 1};
    const float inertia_diag[3] = {9.416556729130406e-6f, 9.644051701582312e-6f, 1.745951732253285e-5f};
    const float inertia_inv_diag[3] = {106195.93007988465f, 103690.85846314249f, 57275.35197719487f};
    for (int r = 0; r < 4; ++r) {
        const int i = 3 * r;
        p.rotor_positions[i] = positions[i];
        p.rotor_positions[i + 1] = positions[i + 1];
        p.rotor_thrust_directions[i + 2] = 1.0f;
        p.rotor_torque_directions[i + 2] = torque_z[r];
        p.rotor_thrust_coefficients[i] = 0.00352526f;
        p.rotor_thrust_coefficients[i + 1] = 0.01437313f;
        p.rotor_thrust_coefficients[i + 2] = 0.09223048f;
        p.rotor_torque_constants[r] = 4.665e-3f;
        p.rotor_time_constants_rising[r] = 0.05545454545454546f;
        p.rotor_time_constants_falling[r] = 0.24939393939393945f;
    }
    for (int i = 0; i < 3; ++i) {
        p.inertia[4 * i] = inertia_diag[i];
        p.inertia_inverse[4 * i] = inertia_inv_diag[i];
    }
    p.gravity_world[2] = -9.81f;
    p.mass = 0.027f + 0.0017f + 0.0003f + 0.0016f;
    p.action_min = 0.0f;
    p.action_max = 1.0f;
    p.dt = 0.01f;
    p.position_limit = 100000.0f;
    p.velocity_limit = 100000.0f;
    p.angular_velocity_limit = 100000.0f;
    return p;
}

constexpr MdnPhysicsParams kCrazyflie = crazyflie_profile();

}  // namespace mdn

#endif
