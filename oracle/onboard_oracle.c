/*
 * TEST INFRASTRUCTURE ONLY: the CPU checker for the onboard tactical (24)
 * and physics-prior (15) features.
 *
 * Restates the reference device code src/network/onboard_features.cuh:6-519
 * in C11 single precision with libm (cosf, atan2f, ...), keeping its
 * expressions and evaluation order; built without FMA contraction.  The
 * reference pins it with 40 golden values at 5e-5 and output bounds
 * (tests/test_onboard_features.cu:19-39,55-85 of the reference), which
 * tests/test_onboard_oracle.py checks.  Every mission mode of the prior and
 * all 24 tactical outputs are further pinned by closed forms at chosen
 * states, mirror symmetry and a second formulation of the tactical features
 * (tests/test_onboard_prior_pins.py); the cluster y sum's float scan order
 * by near-cancelling clusters (tests/test_onboard_oracle.py).
 *
 * Optional diagnostics (no counterpart in the reference outputs):
 *   diag[0] min_r          closest in-window LiDAR return of elevations 0..3
 *   diag[1] argmin ray     its ray index (head*768 + el*128 + azi), -1 if none
 *   diag[2] min_dx_c       nearest corridor x-centre (30 when none)
 *   diag[3] cluster_count  rays within 1.4 m of that corridor minimum
 *   diag[4] cluster_y_sum  their y centres summed in float in scan order
 */
#include "oracle.h"

#include <math.h>
#include <stdbool.h>

#define OB_PI 3.14159265358979323846f

/* onboard_features.cuh:6-22 */
static float ob_clamp(float x, float lo, float hi) {
    if (isnan(x)) return x;
    return fminf(hi, fmaxf(lo, x));
}
static float ob_obs(float x) {
    return isnan(x) ? 0.0f : (isinf(x) ? copysignf(1000.0f, x) : x);
}
static float ob_mission(float x) {
    return isnan(x) ? 0.0f : (isinf(x) ? copysignf(1.0f, x) : x);
}
static float ob_wrap(float target, float current) {
    const float d = target - current;
    return atan2f(sinf(d), cosf(d));
}
static float ob_norm3(float x, float y, float z) {
    return sqrtf(x * x + y * y + z * z);
}

/* onboard_features.cuh:25-86 */
static void ob_tactical(const float *o, const float *m, float t[24]) {
    const float pi = OB_PI;
    float spool[4], fz[4], tau_z = 0.0f, spool_mean = 0.0f;
    for (int i = 0; i < 4; ++i) {
        spool[i] = ob_clamp(o[16 + i], 0.0f, 1.0f);
        const float thrust = 0.036f + 0.964f * spool[i];
        const float ci = cosf(o[28 + i]);
        fz[i] = thrust * o[24 + i] * ci;
        tau_z += thrust * o[20 + i] * ci;
        spool_mean += spool[i];
    }
    spool_mean *= 0.25f;
    t[0] = fz[1] - fz[3];
    t[1] = fz[2] - fz[0];
    t[2] = 0.5f * tau_z;
    t[3] = 0.25f * (fz[0] + fz[1] + fz[2] + fz[3]) - 0.5f;
    for (int i = 0; i < 4; ++i) t[4 + i] = 2.0f * (spool[i] - spool_mean);

    const float qw = o[6], qx = o[7], qy = o[8], qz = o[9];
    const float bz_x = 2.0f * (qx * qz + qw * qy);
    const float bz_y = 2.0f * (qy * qz - qw * qx);
    const float ct = ob_clamp(1.0f - 2.0f * (qx * qx + qy * qy), -1.0f, 1.0f);
    const float bx_x = 1.0f - 2.0f * (qy * qy + qz * qz);
    const float bx_y = 2.0f * (qx * qy + qw * qz);
    const float yaw = atan2f(bx_y, bx_x), cy = cosf(yaw), sy = sinf(yaw);
    t[8] = cy * bz_y - sy * bz_x;
    t[9] = -sy * bz_y - cy * bz_x;
    t[10] = ct;
    t[11] = ct < 0.20f ? 1.0f : 0.0f;

    const float rx = atanhf(ob_clamp(m[7], -0.995f, 0.995f)) * 20.0f;
    const float ry = atanhf(ob_clamp(m[8], -0.995f, 0.995f)) * 20.0f;
    const float rz = atanhf(ob_clamp(m[9], -0.995f, 0.995f)) * 20.0f;
    t[12] = tanhf((cy * rx + sy * ry) * 0.08f);
    t[13] = tanhf((-sy * rx + cy * ry) * 0.08f);
    t[14] = tanhf(rz * 0.12f);
    t[15] = tanhf(hypotf(rx, ry) * 0.05f);
    t[16] = tanhf((cy * o[3] + sy * o[4]) * 0.15f);
    t[17] = tanhf((-sy * o[3] + cy * o[4]) * 0.15f);
    t[18] = expf(-fmaxf(o[2] - 0.62f, 0.0f));

    /* Ballistic aim of the goal offset, rotated into the body frame by the
     * conjugate quaternion (v' = v + 2u x (u x v + w v), u = -q.xyz). */
    const float dist = fmaxf(ob_norm3(rx, ry, rz), 1.0f);
    const float flight = dist / 20.0f;
    const float wx = rx - o[3] * 0.5f * flight;
    const float wy = ry - o[4] * 0.5f * flight;
    const float wz = rz - o[5] * 0.5f * flight + 0.5f * 9.80665f * flight * flight;
    const float ux = -qx, uy = -qy, uz = -qz;
    const float cx = uy * wz - uz * wy + qw * wx;
    const float cyq = uz * wx - ux * wz + qw * wy;
    const float cz = ux * wy - uy * wx + qw * wz;
    const float bx = wx + 2.0f * (uy * cz - uz * cyq);
    const float by = wy + 2.0f * (uz * cx - ux * cz);
    const float bz = wz + 2.0f * (ux * cyq - uy * cx);
    const float az = ob_clamp(atan2f(by, bx), pi / 12.0f, pi * 5.0f / 12.0f);
    const float el = ob_clamp(atan2f(bz, fmaxf(hypotf(bx, by), 0.2f)), -pi / 6.0f, pi / 6.0f);
    const float err = hypotf(az - o[44], el - o[45]);
    t[19] = (az - pi * 0.25f) / (pi / 6.0f);
    t[20] = el / (pi / 6.0f);
    t[21] = tanhf(err * 2.0f);
    t[22] = (o[46] <= 0.02f && o[47] > 0.01f && err < 0.26f && dist < 34.0f) ? 1.0f : -1.0f;
    t[23] = sinf(atan2f(ry, rx) - pi * 0.25f - yaw);
    for (int i = 0; i < 24; ++i)
        t[i] = isnan(t[i]) ? 0.0f : (isinf(t[i]) ? copysignf(1.0f, t[i]) : t[i]);
}

/* The LiDAR scan of onboard_features.cuh:184-234: rays of both heads at
 * elevations 0..5, all 128 azimuths, in-window ranges 0.35 < r < 11.5. */
typedef struct {
    float min_r, min_r_dx, min_r_dy;
    int min_ray;
    float min_dx_c, cluster_y_sum;
    int cluster_count;
} ob_scan;

/* Body-frame unit vector of ray (head, el, azi), onboard_features.cuh:194-197. */
static void ob_ray_dir(int head, int el, int azi, float d[3]) {
    const float pi = OB_PI;
    const float elev = (head == 0 ? 1.0f : -1.0f) * (pi * el / 30.0f);
    const float azim = pi * (0.25f + azi / 64.0f);
    d[0] = cosf(elev) * cosf(azim);
    d[1] = cosf(elev) * sinf(azim);
    d[2] = sinf(elev);
}

void orc_onboard_ray_dir(int ray, float *xyz) {
    ob_ray_dir(ray / 768, (ray % 768) / 128, ray % 128, xyz);
}

static void ob_ray_world(const float r[9], int head, int el, int azi,
                         float *rwx, float *rwy, float *rwz) {
    float d[3];
    ob_ray_dir(head, el, azi, d);
    *rwx = r[0] * d[0] + r[1] * d[1] + r[2] * d[2];
    *rwy = r[3] * d[0] + r[4] * d[1] + r[5] * d[2];
    *rwz = r[6] * d[0] + r[7] * d[1] + r[8] * d[2];
}

static void ob_lidar_scan(const float *input_obs, const float r[9], float py, ob_scan *s) {
    s->min_r = 30.0f; s->min_r_dx = 0.0f; s->min_r_dy = 0.0f; s->min_ray = -1;
    s->min_dx_c = 30.0f; s->cluster_y_sum = 0.0f; s->cluster_count = 0;
    for (int pass = 0; pass < 2; ++pass)
        for (int head = 0; head < 2; ++head)
            for (int el = 0; el < 6; ++el)
                for (int azi = 0; azi < 128; ++azi) {
                    const float range = ob_obs(input_obs[48 + (head * 16 + el) * 128 + azi]);
                    if (!(range > 0.35f && range < 11.5f)) continue;
                    float rwx, rwy, rwz;
                    ob_ray_world(r, head, el, azi, &rwx, &rwy, &rwz);
                    const float wx = rwx * range, wy = rwy * range, wz = rwz * range;
                    const float x_center = wx + rwx * 1.10f;
                    const float y_center = py + wy + rwy * 1.10f;
                    const bool corridor = fabsf(wz) <= 2.1f && x_center >= -0.35f &&
                                          x_center <= 10.5f && fabsf(y_center) <= 3.5f;
                    if (pass == 0) {
                        if (el < 4 && range < s->min_r) {
                            s->min_r = range; s->min_r_dx = wx; s->min_r_dy = wy;
                            s->min_ray = head * 768 + el * 128 + azi;
                        }
                        if (corridor && x_center < s->min_dx_c) s->min_dx_c = x_center;
                    } else if (corridor && x_center <= s->min_dx_c + 1.4f) {
                        ++s->cluster_count;
                        s->cluster_y_sum += y_center;
                    }
                }
}

/* onboard_features.cuh:88-513 */
static void ob_prior(const float *input_obs, const float *input_mission, float n[15],
                     float *diag) {
    const float pi = OB_PI;
    const float max_installed = 294.2f * 0.85f;
    const float idle_frac = 0.08f;
    const float min_thrust = max_installed * idle_frac;
    const float gravity = 9.80665f;
    const float outer_limit = 2.0f;
    const float inner_limit = pi / 4.0f;
    const float cannon_az_ctr = pi / 4.0f;
    const float cannon_az_half = pi / 6.0f;
    const float cannon_el_lim = pi / 6.0f;
    float o[48], m[10];
    for (int i = 0; i < 48; ++i) o[i] = ob_obs(input_obs[i]);
    for (int i = 0; i < 10; ++i) m[i] = ob_mission(input_mission[i]);
    const float px = o[0], py = o[1], pz = o[2], vx = o[3], vy = o[4], vz = o[5];

    /* Attitude (:105-109): normalised, sign-fixed quaternion. */
    float qnorm = fmaxf(ob_norm3(o[6], o[7], o[8]), 0.0f);
    qnorm = fmaxf(sqrtf(qnorm * qnorm + o[9] * o[9]), 1.0e-8f);
    const float sign = o[6] < 0.0f ? -1.0f : 1.0f;
    const float qw = sign * o[6] / qnorm, qx = sign * o[7] / qnorm;
    const float qy = sign * o[8] / qnorm, qz = sign * o[9] / qnorm;
    const float ox = o[10], oy = o[11], oz = o[12];
    const float omega_norm = ob_norm3(ox, oy, oz);

    /* Arms (:112-123). */
    float spool[4], thrust[4], outer[4], ft[4];
    float total_fz = 0.0f, jammed_yaw_ft = 0.0f, fz[4];
    for (int i = 0; i < 4; ++i) {
        spool[i] = ob_clamp(o[16 + i], 0.0f, 1.0f);
        thrust[i] = max_installed * (idle_frac + (1.0f - idle_frac) * spool[i]);
        outer[i] = atan2f(o[20 + i], o[24 + i]);
        const float inner = o[28 + i];
        fz[i] = thrust[i] * cosf(outer[i]) * cosf(inner);
        ft[i] = thrust[i] * sinf(outer[i]) * cosf(inner);
        total_fz += fz[i];
        jammed_yaw_ft += ft[i];
    }

    /* Mission decode (:124-131). */
    const bool landing = m[1] > 0.75f;
    const bool cargo = m[2] > 0.75f;
    const bool inversion = m[3] > 0.75f && m[0] < -0.25f;
    const bool turbine_out = m[3] > 0.75f && m[2] < -0.25f;
    const bool lateral = m[4] > 0.75f && m[5] > 0.25f;
    const bool slalom = m[4] > 0.75f && !lateral;
    const bool dodge = m[5] > 0.75f;
    const bool arena = m[6] > 0.75f;

    /* Mass and rotation (:132-153). */
    const float fuel = ob_clamp(o[40], 0.0f, 1.0f) * 9.0f;
    const float ammo_mass = ob_clamp(o[47], 0.0f, 4.0f) * 6.0f;
    const bool payload = o[41] > 0.5f;
    const float mass = (arena ? 40.0f : 43.0f) + fuel + ammo_mass + (payload ? 30.0f : 0.0f);
    const float weight = mass * gravity;
    const float r[9] = {
        1.0f - 2.0f * (qy * qy + qz * qz), 2.0f * (qx * qy - qw * qz), 2.0f * (qx * qz + qw * qy),
        2.0f * (qx * qy + qw * qz), 1.0f - 2.0f * (qx * qx + qz * qz), 2.0f * (qy * qz - qw * qx),
        2.0f * (qx * qz - qw * qy), 2.0f * (qy * qz + qw * qx), 1.0f - 2.0f * (qx * qx + qy * qy)};
    const float r00 = r[0], r01 = r[1], r02 = r[2], r10 = r[3], r11 = r[4], r12 = r[5];
    const float r20 = r[6], r21 = r[7], r22 = r[8];
    (void)r01; (void)r11; (void)r12; (void)r02;
    const float body_z_x = 2.0f * (qx * qz + qw * qy);
    const float body_z_y = 2.0f * (qy * qz - qw * qx);
    const float ct = ob_clamp(r22, -1.0f, 1.0f);
    const float yaw = atan2f(r10, r00);
    const float tau_x_actual = fz[1] - fz[3];
    const float tau_y_actual = fz[2] - fz[0];
    const float az_actual = (total_fz * ct - weight) / mass;
    const bool heavy_cargo = cargo && payload;
    const bool landing_like = landing || heavy_cargo;

    /* Targets (:156-183). */
    const float relx = atanhf(ob_clamp(m[7], -0.9995f, 0.9995f)) * 20.0f;
    const float rely = atanhf(ob_clamp(m[8], -0.9995f, 0.9995f)) * 20.0f;
    const float relz = atanhf(ob_clamp(m[9], -0.9995f, 0.9995f)) * 20.0f;
    float tx = (arena || lateral) ? px + relx : 0.0f;
    if (cargo) tx = 15.0f;
    if (slalom) tx = 36.0f;
    const float ty = (arena || lateral) ? py + rely : 0.0f;
    float tz = 8.0f;
    if (landing) tz = 0.60f;
    if (inversion) tz = 14.0f;
    if (cargo || arena) tz = pz + relz;
    float ex = tx, ey = ty, ez = tz;
    const float dx_opp = tx - px, dy_opp = ty - py;
    const float dxy = hypotf(dx_opp, dy_opp);
    const bool valid_d = dxy > 1.0e-3f;
    const float safe_d = valid_d ? dxy : 1.0f;
    const bool intercept = arena && m[0] > 0.75f && m[5] < -0.25f;
    const float desired_range = intercept ? 8.5f : 12.5f;
    float ax = valid_d ? tx - (dx_opp / safe_d) * desired_range : tx;
    float ay = valid_d ? ty - (dy_opp / safe_d) * desired_range : ty;
    const float scale = fminf(16.0f / fmaxf(hypotf(ax, ay), 1.0e-3f), 1.0f);
    ax *= scale; ay *= scale;
    const float pull = ob_clamp((hypotf(px, py) - 21.0f) / 10.0f, 0.0f, 1.0f);
    ax *= 1.0f - pull; ay *= 1.0f - pull;
    const float az_t = pz < 8.0f || vz < -1.0f ? 12.2f : ob_clamp(tz, 8.5f, 12.2f);
    if (arena) { ex = ax; ey = ay; ez = az_t; }
    const float errx = ex - px, erry = ey - py;
    const float horiz_dist = hypotf(errx, erry);

    /* LiDAR passes (:184-239). */
    ob_scan scan;
    ob_lidar_scan(input_obs, r, py, &scan);
    float avoid_x = 0.0f, avoid_y = 0.0f, slalom_speed = 3.8f, nearest_dx = 30.0f;
    if (dodge && scan.min_r < 7.5f) {
        const float min_az = atan2f(scan.min_r_dy, scan.min_r_dx);
        avoid_x = -sinf(min_az) * 2.2f;
        avoid_y = cosf(min_az) * 2.2f;
    }
    const float min_dx_c = scan.min_dx_c;
    const int cluster_count = scan.cluster_count;
    const float cluster_y = scan.cluster_y_sum / fmaxf((float)cluster_count, 1.0f);
    const bool has_slalom_obs = slalom && horiz_dist > 2.5f && min_dx_c < 10.2f &&
                                cluster_count > 0;
    if (has_slalom_obs) {
        nearest_dx = min_dx_c;
        ey = cluster_y >= 0.0f ? -1.85f : 1.85f;
    }
    const float lane_err = fabsf(py - ey);
    float speed_limit = lane_err > 0.55f ? 2.75f : 4.10f;
    if (lane_err > 1.05f) speed_limit = 1.55f;
    if (min_dx_c >= 6.6f && px > 4.0f) speed_limit = 3.10f;
    if (has_slalom_obs) slalom_speed = speed_limit;
    if (slalom && horiz_dist > 3.5f) {
        const float hill = ob_clamp((px - 6.0f) / 30.0f, 0.0f, 1.0f);
        ez = 2.5f * sinf(pi * hill) + 8.0f;
    }
    if (diag) {
        diag[0] = scan.min_r;
        diag[1] = (float)scan.min_ray;
        diag[2] = scan.min_dx_c;
        diag[3] = (float)scan.cluster_count;
        diag[4] = scan.cluster_y_sum;
    }

    const float upx = ex - px, upy = ey - py, upz = ez - pz;
    const float up_horiz = hypotf(upx, upy);
    const bool active_slalom = slalom && nearest_dx < 10.2f && horiz_dist > 3.0f;

    /* Landing / cargo targets (:254-283). */
    const float pad_z = fmaxf(ez, 0.60f), above_pad = pz - pad_z;
    const float horiz_speed = hypotf(vx, vy);
    const float transit_cap = heavy_cargo ? 2.65f : 3.4f;
    const float low_cap = above_pad < 1.2f ? 0.55f : (heavy_cargo ? 1.25f : 1.6f);
    const float max_vxy_land = up_horiz > 1.8f ? transit_cap : low_cap;
    const float kp_land = heavy_cargo ? 0.75f : 1.05f;
    const float des_vx_land = ob_clamp(kp_land * upx, -max_vxy_land, max_vxy_land);
    const float des_vy_land = ob_clamp(kp_land * upy, -max_vxy_land, max_vxy_land);
    const float vz_land_touch = pz > 0.635f ? -0.16f : 0.0f;
    const float vz_land_cargo = ob_clamp(1.6f * (0.64f - pz), -0.30f, 0.18f);
    const float vz_land_low = cargo ? vz_land_cargo : vz_land_touch;
    const float max_desc = cargo ? -0.82f : -1.4f;
    const float vz_land_mid = ob_clamp(-0.70f * above_pad, max_desc, -0.25f);
    const float vz_land_align = ob_clamp(1.2f * (pad_z + 0.90f - pz), -0.30f, 0.60f);
    const float transit_z = heavy_cargo ? fmaxf(1.2f + 0.28f * up_horiz, 2.0f) : 2.0f;
    const float max_desc_trans = heavy_cargo ? -1.05f : -1.6f;
    const float vz_land_trans = ob_clamp(1.3f * (transit_z - pz), max_desc_trans, 1.4f);
    float des_vz_land = above_pad > 1.05f ? vz_land_mid : vz_land_low;
    if ((up_horiz > 0.85f || horiz_speed > 0.65f) && above_pad < 0.95f)
        des_vz_land = vz_land_align;
    if (up_horiz > 1.8f) des_vz_land = vz_land_trans;
    const float max_axy_land = heavy_cargo ? 2.2f : 2.6f;
    const float des_ax_land = ob_clamp(2.4f * (des_vx_land - vx), -max_axy_land, max_axy_land);
    const float des_ay_land = ob_clamp(2.4f * (des_vy_land - vy), -max_axy_land, max_axy_land);
    const float kp_az_land = heavy_cargo ? 5.0f : 4.5f;
    const float kd_az_land = heavy_cargo ? 1.0f : 0.80f;
    const float min_az_land = heavy_cargo ? -1.8f : -2.8f;
    const float des_az_land = ob_clamp(kp_az_land * (des_vz_land - vz) - kd_az_land * az_actual,
                                       min_az_land, 5.5f);

    /* Standard / agile / fault / arena targets (:285-310). */
    const float inv_max_v = up_horiz > 9.0f && fabsf(upz) < 2.5f && ct > 0.90f ? 6.2f : 4.2f;
    const float lat_vx = fabsf(upy) > 1.35f ? 1.45f : 3.8f;
    float max_vx = arena ? 3.2f : 3.0f;
    if (inversion) max_vx = inv_max_v;
    float max_vy = max_vx;
    if (lateral) { max_vx = lat_vx; max_vy = 3.4f; }
    if (slalom) max_vx = 3.5f;
    if (active_slalom) { max_vx = slalom_speed; max_vy = 3.2f; }
    const float max_vz = vz < -2.0f || inversion ? 6.5f : 2.6f;
    const float kp_xy = inversion ? 0.85f : (lateral ? 0.95f : 0.90f);
    const float kp_vx = active_slalom ? 1.25f : kp_xy;
    const float kp_vy = active_slalom ? 1.45f : (lateral ? 1.05f : kp_xy);
    const float des_vx = ob_clamp(kp_vx * upx + avoid_x, -max_vx, max_vx);
    const float des_vy = ob_clamp(kp_vy * upy + avoid_y, -max_vy, max_vy);
    float des_vz = ob_clamp(1.25f * upz, -2.6f, max_vz);
    if ((inversion || arena) && vz < -1.0f) des_vz = fmaxf(des_vz, 0.8f);
    const float kp_ax = active_slalom ? 3.0f : 2.4f;
    const float kp_ay = active_slalom ? 3.0f : 2.6f;
    const float des_ax_std = ob_clamp(kp_ax * (des_vx - vx), -3.8f, 3.8f);
    const float des_ay_std = ob_clamp(kp_ay * (des_vy - vy), -3.8f, 3.8f);
    const float max_az = vz < -1.8f || inversion ? 14.0f : 6.5f;
    const float des_az_std = ob_clamp(3.8f * (des_vz - vz) - 0.80f * az_actual, -4.0f, max_az);
    const float des_ax = landing_like ? des_ax_land : des_ax_std;
    const float des_ay = landing_like ? des_ay_land : des_ay_std;
    const float des_az = landing_like ? des_az_land : des_az_std;

    /* Collective and horizontal force (:312-328). */
    const float tilt = acosf(ct);
    const bool need_headroom = inversion || arena || ct < 0.88f;
    const bool urgent_climb = arena && (pz < 8.5f || vz < -1.2f) && ct > 0.58f;
    const float max_coll = urgent_climb ? 3.95f :
        (need_headroom ? ob_clamp(3.95f - 0.90f * omega_norm - 1.30f * tilt, 2.55f, 3.95f)
                       : 3.95f);
    const float fz_des = ob_clamp((weight + mass * des_az) / fmaxf(ct, 0.45f),
                                  0.10f * weight, max_coll * max_installed);
    const float horiz_scale = urgent_climb ? 0.0f :
        (need_headroom ? ob_clamp(1.0f - 1.5f * fmaxf(tilt - 0.15f, 0.0f), 0.0f, 1.0f) : 1.0f);
    const float tilt_comp = turbine_out ? 0.65f : 0.0f;
    const float damp_v = active_slalom ? 0.8f : 0.4f;
    const float fx_world =
        (mass * des_ax + damp_v * vx - tilt_comp * total_fz * body_z_x) * horiz_scale;
    const float fy_world =
        (mass * des_ay + damp_v * vy - tilt_comp * total_fz * body_z_y) * horiz_scale;
    const float cy = cosf(yaw), sy = sinf(yaw);
    const float max_fh = active_slalom ? 105.0f :
        (lateral ? 125.0f : (heavy_cargo ? 52.0f : 80.0f));
    const float fx_body = ob_clamp(cy * fx_world + sy * fy_world, -max_fh, max_fh);
    const float fy_body = ob_clamp(-sy * fx_world + cy * fy_world, -max_fh, max_fh);

    /* Tilt error in the body frame (:330-339). */
    const float cw_x = body_z_y, cw_y = -body_z_x;
    const float ux = -qx, uy = -qy, uz = -qz;
    const float tt_x = 2.0f * (-uz * cw_y), tt_y = 2.0f * (uz * cw_x);
    const float tt_z = 2.0f * (ux * cw_y - uy * cw_x);
    const float te_x = cw_x + qw * tt_x + (uy * tt_z - uz * tt_y);
    const float te_y = cw_y + qw * tt_y + (uz * tt_x - ux * tt_z);
    const float te_z = qw * tt_z + (ux * tt_y - uy * tt_x);
    const float te_norm = ob_norm3(te_x, te_y, te_z);
    const float tilt_scale = te_norm > 1.0e-5f ? tilt / fmaxf(te_norm, 1.0e-5f) : 0.0f;
    const float e_rx = te_x * tilt_scale, e_ry = te_y * tilt_scale;

    /* Yaw target (:341-348). */
    const bool inv_hold_yaw = (inversion || arena) && (pz < 6.0f || vz < -0.5f || ct < 0.88f);
    const bool opp_bearing_valid = arena && fabsf(m[1]) + fabsf(m[2]) > 0.1f;
    const float opp_bearing = atan2f(m[1], m[2]);
    const float raw_bearing = atan2f(ty - py, tx - px);
    const float target_bearing = opp_bearing_valid ? opp_bearing : raw_bearing;
    const float desired_yaw = arena && horiz_dist > 1.0f && !inv_hold_yaw ?
        target_bearing - cannon_az_ctr : (inv_hold_yaw ? yaw : 0.0f);
    const float yaw_err = ob_wrap(desired_yaw, yaw);

    /* Torques and per-arm commands (:350-393). */
    const float parasite_scale = turbine_out ? 0.35f : 1.0f;
    const float tau_x_par = -0.1625f * fy_body * parasite_scale;
    const float tau_y_par = 0.1625f * fx_body * parasite_scale;
    const float tau_x_net = tau_x_actual + tau_x_par;
    const float tau_y_net = tau_y_actual + tau_y_par;
    const float max_txy = heavy_cargo ? 120.0f : 260.0f;
    const float tau_x_cmd = ob_clamp(95.0f * e_rx - 64.0f * ox - 0.90f * tau_x_net - tau_x_par,
                                     -max_txy, max_txy);
    const float tau_y_cmd = ob_clamp(95.0f * e_ry - 64.0f * oy - 0.90f * tau_y_net - tau_y_par,
                                     -max_txy, max_txy);
    const float tau_z_cmd = ob_clamp(22.0f * yaw_err - 18.0f * oz, -70.0f, 70.0f);
    const float fz_cmd[4] = {
        0.25f * fz_des - tau_y_cmd * 0.5f,
        0.25f * fz_des + tau_x_cmd * 0.5f,
        0.25f * fz_des + tau_y_cmd * 0.5f,
        0.25f * fz_des - tau_x_cmd * 0.5f
    };
    const float yaw_ft = (tau_z_cmd - 0.40f * jammed_yaw_ft) * 0.25f;
    float outer_cmd[4], inner_cmd[4], throttle[4], u_raw[4];
    const float fx_outer = ft[3] - ft[1];
    const float fy_outer = ft[0] - ft[2];
    const float fx_rem = fx_body - fx_outer, fy_rem = fy_body - fy_outer;
    const float max_sin_inner = lateral ? 0.44f :
        (active_slalom ? 0.42f : (heavy_cargo ? 0.22f : 0.32f));
    const float spool_gain = turbine_out ? 10.5f : (heavy_cargo ? 4.5f : 2.4f);
    float max_raw = -INFINITY;
    const bool land_idle = landing && pz <= 0.638f && up_horiz < 0.85f && fabsf(vz) < 0.20f;
    for (int i = 0; i < 4; ++i) {
        const float yaw_alpha = asinf(ob_clamp(yaw_ft / fmaxf(thrust[i], 30.0f), -0.35f, 0.35f));
        outer_cmd[i] = ob_clamp(6.5f * ob_wrap(yaw_alpha, outer[i]), -outer_limit, outer_limit);
        const float urx = i == 0 ? 1.0f : (i == 2 ? -1.0f : 0.0f);
        const float ury = i == 1 ? 1.0f : (i == 3 ? -1.0f : 0.0f);
        const float fr_req = 0.5f * (fx_rem * urx + fy_rem * ury);
        const float sin_in = ob_clamp(fr_req / fmaxf(thrust[i], 40.0f), -max_sin_inner,
                                      max_sin_inner);
        inner_cmd[i] = ob_clamp(asinf(sin_in), -inner_limit * 0.90f, inner_limit * 0.90f);
        const float nominal_cos = fmaxf(cosf(yaw_alpha) * cosf(inner_cmd[i]), 0.70f);
        float target_thrust = fmaxf(fz_cmd[i], 0.0f) / nominal_cos;
        if (land_idle) target_thrust = 0.15f * weight * 0.25f;
        const float u_des = ob_clamp((target_thrust - min_thrust) / (max_installed - min_thrust),
                                     0.0f, 1.0f);
        u_raw[i] = u_des + spool_gain * (u_des - spool[i]);
        max_raw = fmaxf(max_raw, u_raw[i]);
    }
    const float excess = ob_clamp(max_raw - 1.0f, 0.0f, urgent_climb ? 0.10f : 0.45f);
    for (int i = 0; i < 4; ++i)
        throttle[i] = ob_clamp(u_raw[i] - (need_headroom ? excess : 0.0f), 0.0f, 1.0f);

    /* Inverted recovery (:394-405). */
    const bool inv_mode = ct < 0.20f;
    if (inv_mode) {
        const float inv_rx = te_norm > 1.0e-5f ? e_rx : tilt;
        const float tx_inv = 130.0f * inv_rx - 52.0f * ox;
        const float ty_inv = 130.0f * e_ry - 52.0f * oy;
        const float arm_mom[4] = {-ty_inv, tx_inv, ty_inv, -tx_inv};
        for (int i = 0; i < 4; ++i) {
            throttle[i] = arm_mom[i] > 12.0f ? 0.58f : 0.0f;
            outer_cmd[i] = ob_clamp(-outer[i] * 6.0f, -outer_limit, outer_limit);
            inner_cmd[i] = 0.0f;
        }
    }

    /* Cannon (:407-431). */
    const float to_x = tx - px, to_y = ty - py, to_z = tz - pz;
    const float dist = fmaxf(ob_norm3(to_x, to_y, to_z), 1.0f);
    const float flight = dist / 20.0f;
    const float aim_x = to_x - vx * (0.65f * flight);
    const float aim_y = to_y - vy * (0.65f * flight);
    const float aim_z = to_z - vz * (0.65f * flight) + 0.53f * gravity * flight * flight;
    const float cx = uy * aim_z - uz * aim_y + qw * aim_x;
    const float cyq = uz * aim_x - ux * aim_z + qw * aim_y;
    const float cz = ux * aim_y - uy * aim_x + qw * aim_z;
    const float aim_bx = aim_x + 2.0f * (uy * cz - uz * cyq);
    const float aim_by = aim_y + 2.0f * (uz * cx - ux * cz);
    const float aim_bz = aim_z + 2.0f * (ux * cyq - uy * cx);
    const float des_cannon_az = ob_clamp(atan2f(aim_by, aim_bx), cannon_az_ctr - cannon_az_half,
                                         cannon_az_ctr + cannon_az_half);
    const float des_cannon_el = ob_clamp(atan2f(aim_bz, fmaxf(hypotf(aim_bx, aim_by), 0.2f)),
                                         -cannon_el_lim, cannon_el_lim);
    const float aim_err = hypotf(ob_wrap(des_cannon_az, o[44]), des_cannon_el - o[45]);
    const bool fire = arena && !inv_mode && o[46] <= 0.02f && o[47] > 0.01f &&
                      aim_err < 0.28f && dist < 34.0f;
    const bool cannon = arena && !inv_mode;
    float norm_az = cannon ?
        ob_clamp((des_cannon_az - cannon_az_ctr) / cannon_az_half, -1.0f, 1.0f) : 0.0f;
    if (inv_mode) norm_az = -1.0f;
    float norm_el = cannon ? ob_clamp(des_cannon_el / cannon_el_lim, -1.0f, 1.0f) : 0.0f;
    float norm_fire = fire ? 0.8f : -0.8f;

    /* Blended-wing-body modes (:433-504). */
    const bool bwb_arena = m[6] > 0.75f && m[4] < -0.25f;
    const bool bwb_cruise = m[4] > 0.75f && m[2] > 0.25f;
    const bool bwb_intercept = m[6] > 0.75f && m[5] > 0.60f;
    const bool bwb_endurance = bwb_cruise && m[0] > 0.25f;
    if (bwb_arena || bwb_cruise || bwb_intercept) {
        const float vb_x = r00 * vx + r10 * vy + r20 * vz;
        const float vb_y = r01 * vx + r11 * vy + r21 * vz;
        const float brx = atanhf(ob_clamp(m[7], -0.9999f, 0.9999f)) * 20.0f;
        const float bry = atanhf(ob_clamp(m[8], -0.9999f, 0.9999f)) * 20.0f;
        const float brz = atanhf(ob_clamp(m[9], -0.9999f, 0.9999f)) * 20.0f;
        float btx = px + brx, bty = py + bry, btz = pz + brz;
        const float rxy = hypotf(px, py);
        const float pull_b = ob_clamp((rxy - 235.0f) / 45.0f, 0.0f, 0.85f);
        if (arena && rxy > 235.0f) { btx *= 1.0f - pull_b; bty *= 1.0f - pull_b; }
        if (arena) btz = ob_clamp(btz, 28.0f, 135.0f);
        const float gx = btx - px, gy = bty - py, gz = btz - pz;
        const float gdist = fmaxf(ob_norm3(gx, gy, gz), 1.0f);
        const float desired_yaw_b = atan2f(gy, gx);
        const float gs = hypotf(vx, vy);
        const float course_yaw = gs > 2.5f ? atan2f(vy, vx) : yaw;
        const float course_err = ob_wrap(desired_yaw_b, course_yaw);
        const float desired_speed = bwb_endurance ? 18.5f :
            (arena ? (gdist > 38.0f ? 26.0f : 24.0f) : 22.4f);
        const float speed_err = desired_speed - vb_x;
        const float u_coll = ob_clamp((bwb_endurance ? 0.36f : 0.44f) + 0.065f * speed_err +
                                      0.018f * gz, 0.12f, 0.90f);
        const float roll_right = atan2f(r21, r22);
        const float desired_roll = ob_clamp(-1.35f * course_err, -0.55f, 0.55f);
        const float diff_u = ob_clamp(0.90f * (desired_roll - roll_right) - 0.34f * ox,
                                      -0.45f, 0.45f);
        const float u0 = ob_clamp(u_coll + diff_u, 0.05f, 1.0f);
        const float u1 = ob_clamp(u_coll - diff_u, 0.05f, 1.0f);
        throttle[0] = throttle[2] = u0;
        throttle[1] = throttle[3] = u1;
        const float pitch_up = asinf(ob_clamp(r20, -1.0f, 1.0f));
        const float climb_des = ob_clamp(0.42f * gz, -5.0f, 5.0f);
        const float climb_err = climb_des - vz;
        const float cos_bank = cosf(roll_right), sin_bank = sinf(roll_right);
        const float gamma_des = atan2f(climb_des, fmaxf(gs, 14.0f));
        float desired_pitch = ob_clamp(0.062831853f + 0.75f * gamma_des +
            0.035f * climb_err + 0.09f * (1.0f - fmaxf(cos_bank, 0.5f)), -0.15f, 0.25f);
        if (vb_x < 15.5f) desired_pitch = fminf(desired_pitch, 0.02f);
        const float theta_dot = 2.20f * (desired_pitch - pitch_up);
        const float psi_dot = (gravity / fmaxf(vb_x, 12.0f)) *
            tanf(ob_clamp(-roll_right, -0.75f, 0.75f)) + 0.35f * course_err;
        const float q_up = cos_bank * theta_dot - sin_bank * psi_dot;
        const float r_left = sin_bank * theta_dot + cos_bank * psi_dot;
        const float gimbal = pi / 6.0f;
        inner_cmd[0] = ob_clamp(0.85f * (q_up + oy) + 0.03f, -gimbal, gimbal);
        inner_cmd[1] = ob_clamp(-0.65f * (r_left - oz) - 0.025f * vb_y, -gimbal, gimbal);
        inner_cmd[2] = inner_cmd[3] = 0.0f;
        for (int i = 0; i < 4; ++i) outer_cmd[i] = 0.0f;
        const float oppx = brx - vx * 0.10f, oppy = bry - vy * 0.10f, oppz = brz - vz * 0.10f;
        const float bdist = fmaxf(ob_norm3(oppx, oppy, oppz), 1.0f);
        const bool head_on = bwb_arena && btx * px + bty * py < -800.0f && bdist > 45.0f;
        const float closing = head_on ? 75.0f + 2.0f * fmaxf(vb_x, 0.0f) : 75.0f;
        const float bflight = bdist / closing;
        const float bax = oppx, bay = oppy;
        const float baz = oppz + (head_on ? -vz * (0.85f * bflight) : 0.0f) +
                          0.50f * gravity * bflight * bflight;
        const float bbx = r00 * bax + r10 * bay + r20 * baz;
        const float bby = r01 * bax + r11 * bay + r21 * baz;
        const float bbz = r02 * bax + r12 * bay + r22 * baz;
        const float b_az = ob_clamp(atan2f(bby, fmaxf(bbx, 0.2f)), -pi / 6.0f, pi / 6.0f);
        const float b_el = ob_clamp(atan2f(bbz, fmaxf(hypotf(bbx, bby), 0.2f)),
                                    -cannon_el_lim, cannon_el_lim);
        const float b_err = hypotf(ob_wrap(b_az, o[44]), b_el - o[45]);
        const bool b_fire = arena && o[46] <= 0.02f && o[47] > 0.01f && b_err < 0.045f &&
                            bdist < 165.0f && bbx > 0.0f;
        norm_az = arena ? ob_clamp(b_az / (pi / 6.0f), -1.0f, 1.0f) : 0.0f;
        norm_el = arena ? ob_clamp(b_el / cannon_el_lim, -1.0f, 1.0f) : 0.0f;
        norm_fire = b_fire ? 0.8f : -0.8f;
    }

    /* Normalised action (:505-512). */
    for (int i = 0; i < 4; ++i) {
        n[i] = ob_clamp(throttle[i] * 2.0f - 1.0f, -1.0f, 1.0f);
        n[4 + i] = ob_clamp(outer_cmd[i] / outer_limit, -1.0f, 1.0f);
        n[8 + i] = ob_clamp(inner_cmd[i] / inner_limit, -1.0f, 1.0f);
    }
    n[12] = norm_az;
    n[13] = norm_el;
    n[14] = norm_fire;
}

/* onboard_features.cuh:515-519 */
void orc_onboard_env(const float *obs, const float *mission,
                     float *tactical24, float *prior15, float *diag5) {
    ob_tactical(obs, mission, tactical24);
    ob_prior(obs, mission, prior15, diag5);
}
