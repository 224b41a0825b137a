"""Writes the golden fixtures in tests/golden/ (run in the build container).

Every expected value here comes from installed libraries -- torch's own
torch.optim.AdamW(foreach=False) and CPU tensor ops, and numpy -- never from
this repository's oracle and never from the MORPH sources.  The cases follow
the reference's tests and BASELINE configs:
  * config1.json: BASELINE config 1 (6 FP32 tensors, 10 steps, wd 0.1 on 2-D
    only) through torch.optim.AdamW: SHA-256 of the final masters and moments
    plus a strided sample of each.
  * adamw_exact_sqrt.npz: torch.optim.AdamW with beta2 = 0 and gradients of
    at most 12 significant bits, so every sqrt in the step is exact and the
    expected masters are free of sqrt rounding (bit-exact target).
  * state_cache_kat.npz: the explicit vectors of tests/test_state_cache.py:21-46
    (w = (1, -2, .5); t = 1 grad (2, -1, .5) clip .25; t = 3 grad (-.3, 1.2, 5)
    clip .1; lr .003; chunk 2) run through the op sequence of
    streamtrain/disk.py:209-215 with torch CPU ops.
  * f16_cases.npz: float32 boundary values and numpy's float16 rounding of them.
  * loss_scale.json: the reference's known answer (tests/test_fp16.py:59-72,
    scales [128, 64]) and the BASELINE config 4 sequence.
"""
import hashlib
import json
import math
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent

CONFIG1_SHAPES = [(256, 64), (64, 256), (256,), (512, 256), (256, 512), (512,)]
CONFIG1 = dict(lr=3e-4, betas=(0.9, 0.95), eps=1e-8, wd_2d=0.1, steps=10, master_seed=0,
               grad_seed_base=1000, master_std=0.02, grad_std=1e-3)


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def config1_inputs():
    """Masters N(0, .02) seed 0; grads N(0, 1e-3) seed 1000 + t (t = 1..10)."""
    gen = torch.Generator().manual_seed(CONFIG1["master_seed"])
    masters = [torch.randn(s, generator=gen) * CONFIG1["master_std"] for s in CONFIG1_SHAPES]

    def grads(t):
        g = torch.Generator().manual_seed(CONFIG1["grad_seed_base"] + t)
        return [torch.randn(s, generator=g) * CONFIG1["grad_std"] for s in CONFIG1_SHAPES]
    return masters, grads


def make_config1():
    masters, grads = config1_inputs()
    params = [torch.nn.Parameter(m.clone()) for m in masters]
    groups = [dict(params=[p for p in params if p.ndim == 2], weight_decay=CONFIG1["wd_2d"]),
              dict(params=[p for p in params if p.ndim == 1], weight_decay=0.0)]
    opt = torch.optim.AdamW(groups, lr=CONFIG1["lr"], betas=CONFIG1["betas"], eps=CONFIG1["eps"],
                            foreach=False)
    for t in range(1, CONFIG1["steps"] + 1):
        for p, g in zip(params, grads(t)):
            p.grad = g
        opt.step()
    out = dict(config=CONFIG1, shapes=CONFIG1_SHAPES, tensors=[])
    for p in params:
        st = opt.state[p]
        w, m, v = (p.detach().numpy().ravel(), st["exp_avg"].numpy().ravel(),
                   st["exp_avg_sq"].numpy().ravel())
        idx = np.arange(0, w.size, 997)
        out["tensors"].append(dict(
            sha_w=sha(w), sha_m=sha(m), sha_v=sha(v), sample_index=idx.tolist(),
            sample_w=w[idx].tolist(), sample_m=m[idx].tolist(), sample_v=v[idx].tolist(),
            step=float(st["step"])))
    (HERE / "config1.json").write_text(json.dumps(out))


def twelve_bit(x):
    """Round to 12 significant bits so x*x is exact in binary32."""
    m, e = np.frexp(x.astype(np.float64))
    return np.ldexp(np.round(m * 4096) / 4096, e).astype(np.float32)


def make_exact_sqrt():
    rng = np.random.RandomState(7)
    cases = {}
    for name, beta1, wd in (("b1_0.9_wd", 0.9, 0.1), ("b1_0.3_nowd", 0.3, 0.0)):
        n, steps, lr = 257, 4, 1e-2
        w0 = (rng.randn(n) * .02).astype(np.float32)
        grads = [twelve_bit((rng.randn(n) * 1e-2).astype(np.float32)) for _ in range(steps)]
        grads[1][:5] = 0.0  # exercises denominators equal to eps
        p = torch.nn.Parameter(torch.from_numpy(w0.copy()))
        opt = torch.optim.AdamW([p], lr=lr, betas=(beta1, 0.0), eps=1e-8, weight_decay=wd,
                                foreach=False)
        for g in grads:
            p.grad = torch.from_numpy(g.copy())
            opt.step()
        st = opt.state[p]
        cases[name + "_w0"] = w0
        cases[name + "_grads"] = np.stack(grads)
        cases[name + "_w"] = p.detach().numpy().copy()
        cases[name + "_m"] = st["exp_avg"].numpy().copy()
        cases[name + "_v"] = st["exp_avg_sq"].numpy().copy()
        cases[name + "_hyper"] = np.array([lr, beta1, 0.0, 1e-8, wd, steps], np.float64)
    np.savez(HERE / "adamw_exact_sqrt.npz", **cases)


def make_state_cache_kat():
    state = np.stack([np.array([1.0, -2.0, 0.5], np.float32), np.zeros(3, np.float32),
                      np.zeros(3, np.float32)])
    snapshots = []
    for step, grad, clip in ((1, [2.0, -1.0, 0.5], 0.25), (3, [-0.3, 1.2, 5.0], 0.1)):
        lr, chunk = 0.003, 2
        gradient = torch.tensor(grad, dtype=torch.float32)
        for start in range(0, 3, chunk):
            end = min(start + chunk, 3)
            weight, first, second = [torch.from_numpy(state[i, start:end].copy()) for i in range(3)]
            g = gradient.flatten()[start:end] * clip
            first.lerp_(g, .1)
            second.mul_(.999).addcmul_(g, g, value=.001)
            denominator = second.sqrt().div_(math.sqrt(1 - .999 ** step)).add_(1e-8)
            weight.mul_(1 - lr * .01).addcdiv_(first, denominator, value=-lr / (1 - .9 ** step))
            state[:, start:end] = np.stack((weight.numpy(), first.numpy(), second.numpy()))
        snapshots.append(state.copy())
    np.savez(HERE / "state_cache_kat.npz", after_t1=snapshots[0], after_t3=snapshots[1])


def make_f16_cases():
    special = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, -65520.0, 1e9,
                        6.103515625e-05, 6.097555160522461e-05, 5.960464477539063e-08,
                        2.980232238769531e-08, 2.9802326e-08, 1e-10, 0.1, 1 / 3,
                        2049.0, 2051.0, 4097.0, np.inf, -np.inf], np.float32)
    rng = np.random.RandomState(3)
    bits = rng.randint(0, 2 ** 32, size=20000, dtype=np.uint64).astype(np.uint32)
    rand = bits.view(np.float32)
    rand = rand[np.isfinite(rand)]
    scaled = (rng.randn(10000) * np.exp(rng.uniform(-20, 12, 10000))).astype(np.float32)
    x = np.concatenate([special, rand, scaled])
    with np.errstate(over="ignore"):  # overflow to inf is the expected rounding
        f16 = x.astype(np.float16)
    np.savez(HERE / "f16_cases.npz", x=x, f16_bits=f16.view(np.uint16))


def make_loss_scale():
    data = dict(
        reference_kat=dict(source="tests/test_fp16.py:59-72", initial=128.0, events=["overflow"],
                           scales_seen=[128.0, 64.0], stored_scale=64.0),
        config4=dict(initial=65536.0, growth_interval=2000, steps=16, overflow_steps=[3, 7, 12],
                     scale_before_step=[65536.0] * 3 + [32768.0] * 4 + [16384.0] * 5 +
                     [8192.0] * 4, final_scale=8192.0),
    )
    (HERE / "loss_scale.json").write_text(json.dumps(data, indent=1))


if __name__ == "__main__":
    torch.set_num_threads(1)
    make_config1()
    make_exact_sqrt()
    make_state_cache_kat()
    make_f16_cases()
    make_loss_scale()
    print("wrote", sorted(p.name for p in HERE.iterdir() if p.suffix in (".json", ".npz")))
