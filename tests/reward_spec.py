"""The walk-to-line reward of one control step, written out in fp64 from the reference's task
definition (src/g1_env.cu:164-199), and hand-built states on which it is known in closed form.

Used as an independent check of both the oracle and the GPU path. The states are airborne, so no
contact acts. Their joints sit exactly at the PD target of the step's action, with zero joint
velocity, so the PD torque and the energy term are zero to rounding. Linear velocity is then
constant over the step (free fall), and the orientation is unchanged without angular velocity.
So the reward follows from the step's end state alone.
"""
import numpy as np

import g1_model as gm

CMD_VX, X_FIN, ALIVE_Z, ALIVE_UP = 0.8, 5.0, 0.45, 0.5


def upright(qpos):
    """z component of the base's body z axis: quat2mat(q)[2][2] = 1 - 2 (x^2 + y^2)."""
    x, y = qpos[..., 4].astype(np.float64), qpos[..., 5].astype(np.float64)
    return 1.0 - 2.0 * (x * x + y * y)


def reward_spec(qp_end, qv_end, vx_mean, act, prev_act, step_before, energy=0.0):
    """(reward, done) of one control step from the state after its last substep.

    alive = z >= 0.45 and up >= 0.5; alive reward 1 + clip(vx_mean, 0, 0.8) upc - 0.2 |vy| -
    0.05 |wz| + 0.3 upc - 0.5 |z - 0.78| - 0.005 min(sum (a - a_prev)^2, 10) - 1e-4 energy,
    upc = clip(up, 0, 1); a fall scores -5; crossing x >= 5 alive adds 50; done = fall or finish or
    the 1000th step of the episode."""
    qp, qv = np.asarray(qp_end, np.float64), np.asarray(qv_end, np.float64)
    up = upright(qp)
    alive = (qp[..., 2] >= ALIVE_Z) & (up >= ALIVE_UP)
    upc = np.clip(up, 0.0, 1.0)
    pen = np.minimum(((np.asarray(act, np.float64) - np.asarray(prev_act, np.float64)) ** 2).sum(-1), 10.0)
    r = (1.0 + np.clip(vx_mean, 0.0, CMD_VX) * upc - 0.2 * np.abs(qv[..., 1]) - 0.05 * np.abs(qv[..., 5])
         + 0.3 * upc - 0.5 * np.abs(qp[..., 2] - 0.78) - 0.005 * pen - 1e-4 * energy)
    r = np.where(alive, r, -5.0)
    won = alive & (qp[..., 0] >= X_FIN)
    r = r + 50.0 * won
    done = (~alive) | won | (np.asarray(step_before) + 1 >= 1000)
    return r, done


def _quat_about_x(deg):
    a = np.deg2rad(deg)
    return np.array([np.cos(a / 2), np.sin(a / 2), 0.0, 0.0], np.float32)


def crafted_cases(seed=0):
    """Worlds whose step reward is known in closed form, plus the three termination causes.

    Returns dict(qp, qv, pa, steps, act, names) in float32/int32. Every alive world is airborne
    (pelvis 0.3 m above its standing height) and keeps its orientation; the cases vary one term at
    a time: forward speed below, above and against the command (clip at 0.8 and at 0),
    lateral speed, a 30 degree roll (upc = cos 30), yaw rate, vertical speed, an action change
    (penalty 0.005 * 2) and a large one (penalty clipped at 10). The done cases: the 1000th step,
    crossing the finish line upright, a pelvis below 0.45 m and a 70 degree roll."""
    stand = gm.qpos_stand.astype(np.float32)
    names = ["vx 0.5 vy 0.3", "vx 1.2 (capped) vy -0.2", "vx -0.4 (clipped)", "roll 30 vx 0.6",
             "yaw rate 0.2", "vz 0.7", "action change", "action change clipped", "timeout",
             "finish line", "fallen (height)", "fallen (tilt)"]
    n = len(names)
    qp = np.tile(stand, (n, 1))
    qp[:, 2] += 0.3
    qv = np.zeros((n, 35), np.float32)
    pa = np.zeros((n, 29), np.float32)
    steps = np.full(n, 17, np.int32)
    act = np.zeros((n, 29), np.float32)
    qv[0, 0], qv[0, 1] = 0.5, 0.3
    qv[1, 0], qv[1, 1] = 1.2, -0.2
    qv[2, 0] = -0.4
    qp[3, 3:7] = _quat_about_x(30.0)
    qv[3, 0] = 0.6
    qv[4, 0], qv[4, 5] = 0.3, 0.2
    qv[5, 0], qv[5, 2] = 0.1, 0.7
    rng = np.random.default_rng(seed)
    a = rng.uniform(-0.3, 0.3, 29).astype(np.float32)
    d = rng.normal(size=29)
    d *= np.sqrt(2.0 / (d ** 2).sum())
    act[6], pa[6] = a, (a - d).astype(np.float32)
    act[7], pa[7] = a, (a - 1.2 * np.sign(rng.normal(size=29))).astype(np.float32)
    for w in (6, 7):   # joints at the step's PD target: zero PD torque
        qp[w, 7:] = np.clip(np.float32(0.5) * act[w] + stand[7:], gm.act_ctrl_lo, gm.act_ctrl_hi)
    steps[8] = 999
    qv[8, 0] = 0.2
    qp[9, 0] = 5.2
    qv[9, 0] = 0.4
    qp[10, 2] = 0.30
    qp[11, 3:7] = _quat_about_x(70.0)
    return dict(qp=qp, qv=qv, pa=pa, steps=steps, act=act, names=names)
