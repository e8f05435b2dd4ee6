"""Flow-matching UniPC multistep sampler (solver order 2, B(h) = expm1, predict x0).

Restates the sampler the reference drives its denoise loop with
(wan/utils/fm_solvers_unipc.py:22-802 as configured at inference_neuron_ti2v.py:504-509:
num_train_timesteps 1000, shift 1 at construction, set_timesteps(steps, shift=5.0);
device variant models/device_unipc.py:24-122), without diffusers:

  construction   sigmas = 1 - linspace(1, 1/N, N)[::-1]          (fm_solvers_unipc.py:115-123)
  set_timesteps  sigmas = linspace(sigma_max, sigma_min, n+1)[:-1], shifted by
                 s*sig/(1 + (s-1)*sig), timesteps = sigmas*N (int64), final sigma 0 (:162-230)
  convert        x0 = x - sigma * v                                  (:281-343)
  UniP (bh2)     x_t = (sig_t/sig_s0) x - alpha_t h_phi_1 m0 - alpha_t B_h sum(rho_p D1)  (:352-486)
  UniC (bh2)     corrector with rho_c = solve(R, b)                  (:488-628)
  step           corrector (from the 2nd step), history shift, predictor; the order
                 warms up 1 -> 2 and drops to 1 on the last step (:657-741)

Scalar coefficients are computed on the host in float32 tensors as the reference
computes them; the tensor arithmetic (linear combinations of the sample and the
stored model outputs) runs on the sample's device, so a step needs no
device-to-host copy.
"""
from typing import List, Optional

import numpy as np
import torch


class FlowUniPC:
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

    # lambda(sigma) = log(alpha) - log(sigma), alpha = 1 - sigma
    def _lambda(self, i: int):
        sigma = self.sigmas[i]
        alpha = 1 - sigma
        return torch.log(alpha) - torch.log(sigma), alpha, sigma

    def _coeffs(self, h: torch.Tensor, rks: List[float]):
        hh = -h
        h_phi_1 = torch.expm1(hh)
        h_phi_k = h_phi_1 / hh - 1
        B_h = torch.expm1(hh)
        factorial_i = 1
        R, b = [], []
        rks_t = torch.tensor(rks)
        for i in range(1, len(rks) + 1):
            R.append(torch.pow(rks_t, i - 1))
            b.append(h_phi_k * factorial_i / B_h)
            factorial_i *= i + 1
            h_phi_k = h_phi_k / hh - 1 / factorial_i
        return torch.stack(R), torch.tensor(b), h_phi_1, B_h

    def _predictor(self, x: torch.Tensor, order: int) -> torch.Tensor:
        m = self.model_outputs
        m0 = m[-1]
        lam_t, alpha_t, sigma_t = self._lambda(self.step_index + 1)
        lam_s0, _, sigma_s0 = self._lambda(self.step_index)
        h = lam_t - lam_s0
        rks, d1 = [], []
        for i in range(1, order):
            lam_si, _, _ = self._lambda(self.step_index - i)
            rk = (lam_si - lam_s0) / h
            rks.append(float(rk))
            d1.append((m[-(i + 1)] - m0) / float(rk))
        rks.append(1.0)
        R, b, h_phi_1, B_h = self._coeffs(h, rks)
        x_t = float(sigma_t / sigma_s0) * x - float(alpha_t * h_phi_1) * m0
        if d1:
            rhos = [0.5] if order == 2 else torch.linalg.solve(R[:-1, :-1], b[:-1]).tolist()
            res = sum(r * d for r, d in zip(rhos, d1))
            x_t = x_t - float(alpha_t * B_h) * res
        return x_t.to(x.dtype)

    def _corrector(self, model_t: torch.Tensor, x: torch.Tensor, order: int) -> torch.Tensor:
        m = self.model_outputs
        m0 = m[-1]
        lam_t, alpha_t, sigma_t = self._lambda(self.step_index)
        lam_s0, _, sigma_s0 = self._lambda(self.step_index - 1)
        h = lam_t - lam_s0
        rks, d1 = [], []
        for i in range(1, order):
            lam_si, _, _ = self._lambda(self.step_index - (i + 1))
            rk = (lam_si - lam_s0) / h
            rks.append(float(rk))
            d1.append((m[-(i + 1)] - m0) / float(rk))
        rks.append(1.0)
        R, b, h_phi_1, B_h = self._coeffs(h, rks)
        rhos = [0.5] if order == 1 else torch.linalg.solve(R, b).tolist()
        res = rhos[-1] * (model_t - m0)
        for r, d in zip(rhos[:-1], d1):
            res = res + r * d
        x_t = float(sigma_t / sigma_s0) * x - float(alpha_t * h_phi_1) * m0 - float(alpha_t * B_h) * res
        return x_t.to(x.dtype)

    def step(self, model_output: torch.Tensor, sample: torch.Tensor) -> torch.Tensor:
        """One sampler step: model_output is the flow (velocity) prediction at the current
        timestep for `sample`; returns the sample at the next timestep."""
        if self.num_inference_steps is None:
            raise RuntimeError("call set_timesteps() first")
        if self.step_index >= self.num_inference_steps:
            raise RuntimeError("all timesteps have been stepped")
        x0 = sample - float(self.sigmas[self.step_index]) * model_output
        if self.step_index > 0 and self.last_sample is not None:
            sample = self._corrector(x0, self.last_sample, self.this_order)
        for i in range(self.solver_order - 1):
            self.model_outputs[i] = self.model_outputs[i + 1]
        self.model_outputs[-1] = x0
        this_order = min(self.solver_order, self.num_inference_steps - self.step_index)
        self.this_order = min(this_order, self.lower_order_nums + 1)
        self.last_sample = sample
        prev = self._predictor(sample, self.this_order)
        if self.lower_order_nums < self.solver_order:
            self.lower_order_nums += 1
        self.step_index += 1
        return prev
