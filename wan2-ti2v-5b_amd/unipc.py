"""Flow-matching UniPC sampler (data prediction, B(h) = e^z - 1, order 2) on device tensors.

The reference drives its denoising loop with FlowUniPCMultistepScheduler
(wan/utils/fm_solvers_unipc.py, configured at inference_neuron_ti2v.py:504-509: 1000
training steps, shift 1 at construction, set_timesteps(steps, shift=5.0)), on the device
through models/device_unipc.py.  diffusers is not needed here: this module implements the
sampler from its published definition (UniPC, Zhao et al. 2023, variant "bh2") in the
flow-matching parameterisation alpha = 1 - sigma.

  schedule    sigma on a shifted linear grid s sig / (1 + (s - 1) sig), then a final 0;
              timestep = int(1000 sigma)                       (fm_solvers_unipc.py:115-230)
  lambda      log(alpha / sigma); a step from sigma_a to sigma_b has h = lambda_b - lambda_a
  x0          x0 = x - sigma v, v the DiT's flow prediction    (:281-343)
  phi         with z = -h:  z phi_1(z) = e^z - 1,  phi_{k+1}(z) = (phi_k(z) - 1/k!) / z
  update      x_b = (sigma_b / sigma_a) x_a - alpha_b (e^z - 1) x0_a - alpha_b B sum_m rho_m D_m
              D_m = (x0 at an earlier point m - x0_a) / r_m, r_m = (lambda_m - lambda_a) / h
  UniP        predictor; order 2 uses rho = 1/2                 (:352-486)
  UniC        corrector: the update from the previous point redone with the new x0
              (its D has r = 1), rho = R^-1 b, R_ij = r_j^i, b_i = z phi_{i+1}(z) i! / B   (:488-628)
  order       1 on the first step, 2 after, 1 again on the last  (:657-741)

Arithmetic follows upstream's tensor code operation for operation, including how
PyTorch rounds: a 0-dim fp32 coefficient that multiplies a tensor from the left is
rounded to that tensor's dtype first, while one on the right (the division by r_m)
keeps its fp32 value.  The coefficients are computed on the host in fp32 and handed
to the tensor ops as Python floats already rounded that way, so a step gives the same
bits on the CPU and on the GPU and needs no device-to-host copy.  The reference's
loop keeps the latent in bf16, and so does denoise() (fast_dit.py).
"""
import math
from typing import List, Optional

import numpy as np
import torch


def _left(coeff: torch.Tensor, t: torch.Tensor) -> float:
    """The fp32 0-dim coefficient `coeff` as a left factor of tensor `t`: rounded to t's
    dtype, as type promotion of a 0-dim tensor does."""
    return float(coeff.to(torch.float32).to(t.dtype))


def _phi_terms(z: torch.Tensor, n: int) -> List[torch.Tensor]:
    """[z phi_2(z), ..., z phi_{n+1}(z)] as fp32 0-dim tensors, by the recurrence
    z phi_{k+1}(z) = z phi_k(z) / z - 1/k! started from z phi_1(z) = e^z - 1."""
    terms, t = [], torch.expm1(z) / z - 1
    for k in range(1, n + 1):
        terms.append(t)
        t = t / z - 1 / math.factorial(k + 1)
    return terms


def _bh2_system(h: torch.Tensor, ratios: List[float]):
    """The linear system of a UniPC-bh2 step of size h (lambda units) with history ratios
    r_1 .. r_p (the last is 1): R [p, p] with R_ij = r_j^i, b [p] with
    b_i = z phi_{i+1}(z) i! / B, and B = e^z - 1, for z = -h."""
    z = -h
    big_b = torch.expm1(z)
    r = torch.tensor(ratios)
    rows = torch.stack([torch.pow(r, i) for i in range(len(ratios))])
    rhs = torch.tensor([t * math.factorial(i + 1) / big_b
                        for i, t in enumerate(_phi_terms(z, len(ratios)))])
    return rows, rhs, big_b


class FlowUniPC:
    """The sampler's state: the sigma schedule, the last `solver_order` x0 predictions and
    the previous sample (for the corrector).  step() takes the model's flow prediction at
    the current timestep and returns the sample at the next one."""

    def __init__(self, num_train_timesteps: int = 1000, solver_order: int = 2, shift: float = 1.0):
        self.num_train_timesteps = num_train_timesteps
        self.solver_order = solver_order
        alphas = np.linspace(1, 1 / num_train_timesteps, num_train_timesteps)[::-1].copy()
        sigmas = torch.from_numpy(1.0 - alphas).to(torch.float32)
        sigmas = shift * sigmas / (1 + (shift - 1) * sigmas)
        self.sigma_min = sigmas[-1].item()
        self.sigma_max = sigmas[0].item()
        self.sigmas = sigmas
        self.timesteps = sigmas * num_train_timesteps
        self.num_inference_steps = None

    def set_timesteps(self, num_inference_steps: int, shift: float = 1.0) -> None:
        sigmas = np.linspace(self.sigma_max, self.sigma_min, num_inference_steps + 1).copy()[:-1]
        sigmas = shift * sigmas / (1 + (shift - 1) * sigmas)
        timesteps = sigmas * self.num_train_timesteps
        self.sigmas = torch.from_numpy(np.concatenate([sigmas, [0.0]]).astype(np.float32))
        self.timesteps = torch.from_numpy(timesteps).to(torch.int64)
        self.num_inference_steps = len(timesteps)
        self.model_outputs: List[Optional[torch.Tensor]] = [None] * self.solver_order
        self.lower_order_nums = 0
        self.last_sample = None
        self.step_index = 0
        self.this_order = 1

    def _point(self, i: int):
        """(lambda, alpha, sigma) of schedule point i as fp32 0-dim tensors."""
        sigma = self.sigmas[i]
        alpha = 1 - sigma
        return torch.log(alpha) - torch.log(sigma), alpha, sigma

    def _bh2_update(self, x: torch.Tensor, a: int, order: int,
                    x0_new: Optional[torch.Tensor] = None) -> torch.Tensor:
        """One UniPC-bh2 update of sample x from schedule point a to a + 1, using the stored
        x0 predictions (the newest, m0, belongs to point a).  Without x0_new it is the
        predictor UniP; with x0_new (the prediction at a + 1) the corrector UniC, whose last
        difference is x0_new - m0."""
        m = self.model_outputs
        m0 = m[-1]
        lam_b, alpha_b, sigma_b = self._point(a + 1)
        lam_a, _, sigma_a = self._point(a)
        h = lam_b - lam_a
        ratios, diffs = [], []
        for j in range(1, order):
            r = float((self._point(a - j)[0] - lam_a) / h)
            ratios.append(r)
            diffs.append((m[-(j + 1)] - m0) / r)
        ratios.append(1.0)
        R, rhs, big_b = _bh2_system(h, ratios)
        if x0_new is None:
            if order == 2:
                rho = [0.5]
            elif order > 2:
                rho = torch.linalg.solve(R[:-1, :-1], rhs[:-1]).to(x.dtype).float().tolist()
            else:
                rho = []
        else:
            rho = [0.5] if order == 1 else torch.linalg.solve(R, rhs).to(x.dtype).float().tolist()
            diffs.append(x0_new - m0)
        total = None
        for w, d in zip(rho, diffs):
            total = w * d if total is None else total + w * d
        out = _left(sigma_b / sigma_a, x) * x - _left(alpha_b * big_b, m0) * m0
        if total is not None:
            out = out - _left(alpha_b * big_b, total) * total
        return out.to(x.dtype)

    def step(self, model_output: torch.Tensor, sample: torch.Tensor) -> torch.Tensor:
        """One sampler step: model_output is the flow (velocity) prediction at the current
        timestep for `sample`; returns the sample at the next timestep."""
        if self.num_inference_steps is None:
            raise RuntimeError("call set_timesteps() first")
        i = self.step_index
        if i >= self.num_inference_steps:
            raise RuntimeError("all timesteps have been stepped")
        x0 = sample - _left(self.sigmas[i], model_output) * model_output
        if i > 0 and self.last_sample is not None:
            sample = self._bh2_update(self.last_sample, i - 1, self.this_order, x0_new=x0)
        self.model_outputs = self.model_outputs[1:] + [x0]
        self.this_order = min(self.solver_order, self.num_inference_steps - i, self.lower_order_nums + 1)
        self.last_sample = sample
        nxt = self._bh2_update(sample, i, self.this_order)
        self.lower_order_nums = min(self.lower_order_nums + 1, self.solver_order)
        self.step_index = i + 1
        return nxt
