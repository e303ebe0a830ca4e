"""PPO training of the G1 walk-to-line task on the fused rollout: each iteration runs one
g1_rollout (all N worlds for H control steps on the GPU, trajectories written into torch
buffers in place), then GAE and clipped-PPO epochs in torch on the same buffers.

    python g1.cu_amd/ppo_train.py [--iters 600] [--worlds 8192] [--horizon 32] [--csv out.csv]

The trajectory contract is the reference driver's (scripts/ppo_fused.py:35-44,82-106). The
weights are packed in the ABI's order (hidden layers W, b; mu head W, b; value head W, b;
log_std). The raw observations in O are normalised on the host with the same frozen statistics
the kernel used, and the running statistics are then updated from those raw observations.
Evaluation uses the host-step path (g1_env_reset / g1_env_step) with deterministic mean actions.
The PPO settings are the reference's, so the reward curves are comparable
(models/ppo_ckpt/reward_curve_fused.csv).
"""
import argparse
import csv
import math
import os
import sys
import time
from dataclasses import dataclass

import numpy as np
import torch
import torch.nn as nn

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import g1env  # noqa: E402

OBS, ACT = g1env.OBS_DIM, g1env.ACT_DIM


@dataclass
class PPOSettings:
    lr: float = 3e-4
    gamma: float = 0.99
    lam: float = 0.95
    clip: float = 0.2
    epochs: int = 5
    minibatches: int = 4
    value_coef: float = 0.5
    entropy_coef: float = 0.01
    max_grad_norm: float = 0.5


class GaussianPolicy(nn.Module):
    """Diagonal Gaussian actor with a value head on a shared MLP trunk. The action's log standard
    deviation is a free parameter (not state dependent). packed() lays the parameters out in the
    order g1_rollout reads them."""

    def __init__(self, hidden=(256, 256), activation="tanh", log_std_init=-0.5):
        super().__init__()
        widths = (OBS,) + tuple(hidden)
        self.trunk = nn.ModuleList(nn.Linear(a, b) for a, b in zip(widths[:-1], widths[1:]))
        self.act = torch.tanh if activation == "tanh" else nn.functional.elu
        self.mu_head = nn.Linear(widths[-1], ACT)
        self.v_head = nn.Linear(widths[-1], 1)
        self.log_std = nn.Parameter(torch.full((ACT,), float(log_std_init)))
        self.hidden, self.activation = tuple(hidden), activation

    def forward(self, z):
        for lin in self.trunk:
            z = self.act(lin(z))
        return self.mu_head(z), self.log_std, self.v_head(z).squeeze(-1)

    def packed(self):
        flat = []
        for lin in list(self.trunk) + [self.mu_head, self.v_head]:
            flat += [lin.weight.detach().flatten(), lin.bias.detach()]
        flat.append(self.log_std.detach())
        return torch.cat(flat).contiguous()


class ObsStats:
    """Running mean and variance of raw observations: count, mean and the sum of squared
    deviations, merged batch by batch (Chan et al.'s pairwise update). Starts at mean 0, variance
    1 with a vanishing weight."""

    def __init__(self, dim, device, prior=1e-4):
        self.n = prior
        self.mean = torch.zeros(dim, device=device)
        self.m2 = torch.full((dim,), prior, device=device)

    @property
    def var(self):
        return self.m2 / self.n

    def update(self, x):
        k = x.shape[0]
        bm = x.mean(0)
        bm2 = ((x - bm) ** 2).sum(0)
        d = bm - self.mean
        tot = self.n + k
        self.mean = self.mean + d * (k / tot)
        self.m2 = self.m2 + bm2 + d * d * (self.n * k / tot)
        self.n = tot

    def frozen(self):
        return self.mean.clone().contiguous(), self.var.clone().contiguous()


def normalize(x, mean, var):
    """The kernel's observation normalisation: (x - mean) / sqrt(var + 1e-8), clipped to +-10."""
    return ((x - mean) / torch.sqrt(var + 1e-8)).clamp(-10.0, 10.0)


def collect(env, policy, stats, traj, act_noise=None, reset_noise=None):
    """One fused rollout into traj with the statistics frozen at its start. Returns the normalised
    observations [H, N, 100] and folds the rollout's raw observations into the statistics."""
    mean, var = stats.frozen()
    traj.run(env, policy.packed(), mean, var, act_noise, reset_noise)
    with torch.no_grad():
        nobs = normalize(traj.O, mean, var)
        stats.update(traj.O.reshape(-1, OBS))
    return nobs


def advantages(traj, gamma, lam):
    """Generalised advantage estimates [H, N] and value targets, backward over the horizon with
    episode boundaries from D (a done step does not bootstrap)."""
    H = traj.R.shape[0]
    adv = torch.empty_like(traj.R)
    running = torch.zeros_like(traj.Vlast)
    next_v = traj.Vlast
    for t in range(H - 1, -1, -1):
        keep = 1.0 - traj.D[t]
        delta = traj.R[t] + gamma * keep * next_v - traj.V[t]
        running = delta + gamma * lam * keep * running
        adv[t] = running
        next_v = traj.V[t]
    return adv, adv + traj.V


def ppo_update(policy, opt, nobs, traj, cfg):
    """Clipped-surrogate PPO epochs over the rollout's samples. Returns the last minibatch loss."""
    adv, ret = advantages(traj, cfg.gamma, cfg.lam)
    obs = nobs.reshape(-1, OBS)
    act = traj.A.reshape(-1, ACT)
    old_lp = traj.LP.reshape(-1)
    ret = ret.reshape(-1)
    adv = adv.reshape(-1)
    adv = (adv - adv.mean()) / (adv.std() + 1e-8)
    n = obs.shape[0]
    size = n // cfg.minibatches
    loss = torch.zeros(())
    for _ in range(cfg.epochs):
        order = torch.randperm(n, device=obs.device)
        for s in range(0, n - size + 1, size):
            idx = order[s:s + size]
            mu, log_std, v = policy(obs[idx])
            z = (act[idx] - mu) / log_std.exp()
            lp = (-0.5 * z * z - log_std - 0.5 * math.log(2 * math.pi)).sum(-1)
            ratio = (lp - old_lp[idx]).exp()
            surr = torch.minimum(ratio * adv[idx], ratio.clamp(1 - cfg.clip, 1 + cfg.clip) * adv[idx])
            entropy = (0.5 + 0.5 * math.log(2 * math.pi) + log_std).sum()
            loss = -surr.mean() + cfg.value_coef * (v - ret[idx]).pow(2).mean() - cfg.entropy_coef * entropy
            opt.zero_grad(set_to_none=True)
            loss.backward()
            nn.utils.clip_grad_norm_(policy.parameters(), cfg.max_grad_norm)
            opt.step()
    return float(loss.detach()), float(ret.mean())


@torch.no_grad()
def evaluate(env, policy, stats, steps=400, dt_ctrl=0.02):
    """Deterministic evaluation through the host-step path: every world starts from g1_env_reset
    and acts with the policy mean. A world's run ends at its first done; forward distance is the
    base x travelled until then (pelvis x before the finishing step), fall_rate the fraction of
    worlds that ended, alive steps and mean forward speed per world."""
    device = policy.log_std.device
    obs = torch.from_numpy(env.reset()).to(device)
    x0 = env.qpos_all()[:, 0].astype(np.float64)
    x_last = x0.copy()
    running = np.ones(env.N, bool)
    alive = np.zeros(env.N)
    mean, var = stats.frozen()
    for _ in range(steps):
        mu, _, _ = policy(normalize(obs, mean, var))
        o, _, done = env.step(mu.cpu().numpy())
        x = env.qpos_all()[:, 0].astype(np.float64)
        finished = done.astype(bool)
        alive[running] += 1
        x_last = np.where(running & ~finished, x, x_last)
        running &= ~finished
        if not running.any():
            break
        obs = torch.from_numpy(o).to(device)
    fwd = x_last - x0
    return dict(forward_m=float(fwd.mean()), forward_max_m=float(fwd.max()), fall_rate=float((~running).mean()),
                alive_steps=float(alive.mean()), vx_mean=float((fwd / np.maximum(alive, 1) / dt_ctrl).mean()))


def train(iters, worlds, horizon, seed=1, eval_every=25, eval_steps=400, csv_path=None, log=print):
    torch.manual_seed(seed)
    cfg = PPOSettings()
    rows = []
    with g1env.Env(worlds, substeps=10, pgs_iters=8, seed=seed) as env:
        policy = GaussianPolicy().cuda()
        stats = ObsStats(OBS, "cuda")
        opt = torch.optim.Adam(policy.parameters(), lr=cfg.lr)
        traj = g1env.Trajectory(horizon, worlds)
        env.reset()
        t0 = time.time()
        for it in range(iters):
            nobs = collect(env, policy, stats, traj)
            rew_step = float(traj.R.mean())
            loss, ret = ppo_update(policy, opt, nobs, traj, cfg)
            row = dict(iter=it, reward_per_step=rew_step, ret=ret, loss=loss,
                       steps_per_s=(it + 1) * horizon * worlds / (time.time() - t0))
            if it % eval_every == 0 or it == iters - 1:
                row.update(evaluate(env, policy, stats, steps=eval_steps))
            rows.append(row)
            log(" ".join(f"{k}={v:.4g}" if isinstance(v, float) else f"{k}={v}" for k, v in row.items()))
            if csv_path:
                keys = ["iter", "reward_per_step", "ret", "loss", "forward_m", "forward_max_m", "alive_steps",
                        "fall_rate", "vx_mean", "steps_per_s"]
                with open(csv_path, "w", newline="") as f:
                    wr = csv.DictWriter(f, keys, restval="")
                    wr.writeheader()
                    wr.writerows(rows)
        err = env.check()
        if err:
            raise RuntimeError(f"physics work queue error {err}")
    return rows


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--iters", type=int, default=600)
    ap.add_argument("--worlds", type=int, default=8192)
    ap.add_argument("--horizon", type=int, default=32)
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--eval-every", type=int, default=25)
    ap.add_argument("--eval-steps", type=int, default=400)
    ap.add_argument("--csv", default=None)
    a = ap.parse_args()
    if not torch.cuda.is_available():
        sys.exit("ppo_train.py needs a GPU")
    train(a.iters, a.worlds, a.horizon, a.seed, a.eval_every, a.eval_steps, a.csv,
          log=lambda s: print(s, flush=True))


if __name__ == "__main__":
    main()
