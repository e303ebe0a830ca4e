"""Fully-on-GPU PPO: each iteration one g1_rollout call runs the whole H-step rollout (physics,
policy inference, sampling, reward) on the device and writes the trajectory into torch-owned
buffers in place; torch then does GAE and the PPO update on the same buffers.

Same calling convention as the reference driver (scripts/ppo_fused.py:27-28,35-44,82-106): the
g1_rollout argtypes, the pack_weights order, raw-observation buffers renormalised with the frozen
statistics the kernel used.

    python g1.cu_amd/scripts/ppo_fused.py [iters] [n_worlds] [--smoke]
"""
import ctypes
import os
import sys
import time

import torch
import torch.nn as nn

from ppo import AC, RunNorm, G1Env, evaluate, _lib, _dp  # noqa: F401  (_lib carries the argtypes)

HERE = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def pack_weights(ac):
    """One contiguous device buffer in kernel order: body linears (weight [out,in] row-major, bias),
    mu weight/bias, v weight/bias, log_std (reference: scripts/ppo_fused.py:35-44)."""
    parts = []
    for m in ac.body:
        if isinstance(m, nn.Linear):
            parts += [m.weight.reshape(-1), m.bias]
    parts += [ac.mu.weight.reshape(-1), ac.mu.bias, ac.v.weight.reshape(-1), ac.v.bias, ac.log_std]
    return torch.cat(parts).contiguous()


def rollout(env, ac, norm, H, bufs):
    """Freeze the normaliser, run one fused rollout into bufs; returns normalised observations."""
    fmean, fvar = norm.mean.clone(), norm.var.clone()
    W = pack_weights(ac)
    O, A, LP, V, R, D, Vlast = bufs
    _lib.g1_rollout(env.h, H, _dp(W), _dp(fmean), _dp(fvar), _dp(O), _dp(A), _dp(LP), _dp(V), _dp(R), _dp(D),
                    _dp(Vlast))
    with torch.no_grad():
        nobs = torch.clamp((O - fmean) / torch.sqrt(fvar + 1e-8), -10.0, 10.0)
        norm.update(O.reshape(-1, O.shape[-1]))
    return nobs


def main():
    dev = "cuda"
    smoke = "--smoke" in sys.argv
    args = [a for a in sys.argv[1:] if not a.startswith("--")]
    iters = int(args[0]) if args else (3 if smoke else 1500)
    N = int(args[1]) if len(args) > 1 else (256 if smoke else 8192)
    H = 16 if smoke else 32
    env = G1Env(N, substeps=10, pgs_iters=8, seed=1)
    od, ad = env.obs_dim, env.act_dim
    ac = AC(od, ad).to(dev)
    norm = RunNorm(od, dev)
    opt = torch.optim.Adam(ac.parameters(), lr=3e-4)
    gamma, lam, clip, epochs, mb = 0.99, 0.95, 0.2, 5, 4
    O = torch.zeros(H, N, od, device=dev); A = torch.zeros(H, N, ad, device=dev)
    LP, V, R, D = (torch.zeros(H, N, device=dev) for _ in range(4))
    Vlast = torch.zeros(N, device=dev)
    bufs = (O, A, LP, V, R, D, Vlast)
    env.reset()
    t0 = time.time()
    for it in range(iters):
        nobs = rollout(env, ac, norm, H, bufs)
        adv = torch.zeros_like(R)
        gae = torch.zeros(N, device=dev)
        for t in reversed(range(H)):
            nextv = Vlast if t == H - 1 else V[t + 1]
            delta = R[t] + gamma * nextv * (1 - D[t]) - V[t]
            gae = delta + gamma * lam * (1 - D[t]) * gae
            adv[t] = gae
        ret = adv + V
        b_o, b_a = nobs.reshape(-1, od), A.reshape(-1, ad)
        b_lp, b_adv, b_ret = LP.reshape(-1), adv.reshape(-1), ret.reshape(-1)
        b_adv = (b_adv - b_adv.mean()) / (b_adv.std() + 1e-8)
        n = b_o.shape[0]
        loss_v = 0.0
        for _ in range(epochs):
            idx = torch.randperm(n, device=dev)
            for s in range(0, n, n // mb):
                j = idx[s:s + n // mb]
                mu, std, val = ac(b_o[j])
                dist = torch.distributions.Normal(mu, std)
                lp = dist.log_prob(b_a[j]).sum(-1)
                ratio = (lp - b_lp[j]).exp()
                pl = -torch.min(ratio * b_adv[j], torch.clamp(ratio, 1 - clip, 1 + clip) * b_adv[j]).mean()
                vl = (val - b_ret[j]).pow(2).mean()
                loss = pl + 0.5 * vl - 0.01 * dist.entropy().sum(-1).mean()
                opt.zero_grad()
                loss.backward()
                nn.utils.clip_grad_norm_(ac.parameters(), 0.5)
                opt.step()
                loss_v = loss.item()
        sps = (it + 1) * H * N / (time.time() - t0)
        msg = f"iter {it:4d} rew/step={R.mean().item():7.3f} ret={b_ret.mean().item():7.3f} loss={loss_v:7.3f} sps={sps:.2e}"
        if it % 25 == 0 or it == iters - 1:
            ev = evaluate(env, ac, norm, dev, steps=20 if smoke else 400)
            msg += f" fwd={ev['fwd_mean']:.2f}m ep_len={ev['ep_len_mean']:.1f} fall={ev['fall_rate']:.2f}"
        print(msg, flush=True)
    env.close()
    if smoke:
        print("SMOKE OK: fused on-GPU rollout + PPO update ran end-to-end.")


if __name__ == "__main__":
    main()
