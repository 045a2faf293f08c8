"""DDPM training/sampling wrapper and weight EMA (diffusion/ddpm.py of the reference).

Same schedules, noise_batch / forward_batch / generate_samples semantics. Differences, all on
purpose: no torch.compile (the training step is captured as one HIP graph instead), the
EMA update is a multi-tensor lerp over the floating-point entries of the state dict only
(the reference multiplies every entry by beta, including the int64 ``window_pos`` buffers of
delayed scaling, which integer tensors cannot hold), and ``forward_batch`` accepts explicit
noise/timesteps so tests can replay a step exactly.
"""
from __future__ import annotations

from copy import deepcopy
from math import pi

import torch
import torch.nn.functional as F

from . import _lib


class EWMAWrapper:
    """diffusion/ddpm.py:10-28."""

    def __init__(self, model: torch.nn.Module, beta: float = 0.9999):
        self.beta = beta
        self.model = deepcopy(model)
        self.model.eval()
        self._pairs: list[tuple[list[torch.Tensor], list[torch.Tensor]]] | None = None

    def _float_entries(self, model: torch.nn.Module):
        ema_sd = self.model.state_dict()
        src_sd = model.state_dict()
        ema, src, ema_int, src_int = [], [], [], []
        for key, ev in ema_sd.items():
            mv = src_sd[key]
            if ev.is_floating_point():
                ema.append(ev)
                src.append(mv)
            else:
                ema_int.append(ev)
                src_int.append(mv)
        return ema, src, ema_int, src_int

    @torch.no_grad()
    def update(self, model: torch.nn.Module) -> None:
        """ema = beta * ema + (1 - beta) * model for every floating-point entry; integer
        buffers (window positions) are copied."""
        ema, src, ema_int, src_int = self._float_entries(model)
        if ema:
            torch._foreach_mul_(ema, self.beta)
            torch._foreach_add_(ema, src, alpha=1.0 - self.beta)
        for e, s in zip(ema_int, src_int):
            e.copy_(s)

    @torch.no_grad()
    def __call__(self, *args, **kwds):
        return self.model(*args, **kwds)


def make_schedule(max_t: int, schedule_type: str):
    """diffusion/ddpm.py:123-175: (alphas, alpha_bars, betas, q_vars, p_vars), float32."""
    if schedule_type == "linear":
        scale = max_t / 1000
        betas = torch.linspace(1e-4 / scale, 0.02 / scale, steps=max_t, dtype=torch.float64)
        alphas = 1.0 - betas
        alpha_bars = torch.cumprod(alphas, dim=-1)
    elif schedule_type == "cosine":
        s = 0.008
        t = torch.linspace(0, max_t, max_t + 1, dtype=torch.float64) / max_t
        alphas_cumprod = torch.cos((t + s) / (1 + s) * pi * 0.5) ** 2
        alphas_cumprod = alphas_cumprod / alphas_cumprod[0]
        betas = torch.clip(1 - (alphas_cumprod[1:] / alphas_cumprod[:-1]), 0, 0.999)
        alphas = 1.0 - betas
        alpha_bars = torch.cumprod(alphas, dim=-1)
    else:
        raise ValueError(schedule_type)
    alpha_bars_prev = torch.concat([torch.tensor(1.0, dtype=torch.float64)[None], alpha_bars[:-1]])
    posterior_variance = betas * (1.0 - alpha_bars_prev) / (1.0 - alpha_bars)
    q_posterior_variance = torch.concat([posterior_variance[1:2], posterior_variance[1:]])
    p_posterior_variance = torch.concat([posterior_variance[1:2], betas[1:]])
    return (alphas.float(), alpha_bars.float(), betas.float(), q_posterior_variance.float(),
            p_posterior_variance.float())


class DiffusionWrapper:
    """diffusion/ddpm.py:31-215."""

    def __init__(self, model, schedule_type: str, max_t: int, in_dim: int, device: str = "cuda",
                 vlb_scale: float = 0.001):
        self.device = torch.device(device)
        alphas, alpha_bars, betas, q_vars, p_vars = make_schedule(max_t, schedule_type)
        self.alphas = alphas.to(self.device)
        self.alpha_bars = alpha_bars.to(self.device)
        self.betas = betas.to(self.device)
        self.q_vars = q_vars.to(self.device)
        self.p_vars = p_vars.to(self.device)
        self.recipsqrt_a = 1.0 / self.alphas.sqrt()
        self.noise_coeff = self.betas / (1.0 - self.alpha_bars).sqrt()
        self.max_t = max_t
        self.in_dim = in_dim
        self.model = model

    @torch.no_grad()
    def _denoise_step(self, samples, t_val: int, recipsqrt_a_t, noise_coeff_t, beta_t, q_var_t):
        t_tensor = torch.full((samples.shape[0],), t_val, device=samples.device)
        with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
            eps_pred = self.model(samples, t_tensor)
        samples = recipsqrt_a_t * (samples - noise_coeff_t * eps_pred)
        if t_val > 0:
            samples += torch.randn_like(samples) * beta_t.sqrt()
        return samples

    @torch.no_grad()
    def generate_samples(self, n_samples: int) -> torch.Tensor:
        samples = torch.randn((n_samples, 3, self.in_dim, self.in_dim), device=self.device)
        samples = samples.to(memory_format=torch.channels_last)
        for idx in reversed(range(self.max_t)):
            samples = self._denoise_step(
                samples, idx, self.recipsqrt_a[idx][..., None, None, None],
                self.noise_coeff[idx][..., None, None, None], self.betas[idx][..., None, None, None],
                self.q_vars[idx][..., None, None, None])
        return samples.clamp(-1.0, 1.0)

    def noise_batch(self, x: torch.Tensor, t: int | torch.Tensor | None = None,
                    eps: torch.Tensor | None = None):
        """(x_t, x_0, eps, t): x_t = sqrt(abar_t) x_0 + sqrt(1 - abar_t) eps (ddpm.py:177-207)."""
        if t is None:
            t_tens = torch.randint(low=0, high=self.max_t, size=(len(x),), device=self.device)
        elif isinstance(t, int):
            t_tens = torch.full((len(x),), device=self.device, fill_value=t)
        else:
            t_tens = t
        if eps is None:
            eps = torch.randn_like(x, device=self.device)
        alpha_bar = self.alpha_bars[t_tens][..., None, None, None]
        return (alpha_bar.sqrt() * x) + ((1.0 - alpha_bar).sqrt() * eps), x, eps, t_tens

    def forward_batch(self, batch: torch.Tensor, t: torch.Tensor | None = None,
                      eps: torch.Tensor | None = None) -> torch.Tensor:
        """Epsilon-prediction MSE (diffusion/ddpm.py:209-215)."""
        noised, _, target, t_tens = self.noise_batch(batch, t, eps)
        eps_pred = self.model(noised, t_tens)
        if eps_pred.is_cuda:
            return mse_loss_hip(eps_pred, target)
        return F.mse_loss(eps_pred, target)


class MSELossHIP(torch.autograd.Function):
    """F.mse_loss(pred, target) (mean) as autocast runs it -- both operands in fp32 -- with the
    loss summed by the HIP library's deterministic two-launch reduction (dpa_mse_loss_f32):
    torch's multi-block reductions record a memset in a captured graph, and replays of the
    training step's graph have returned 0 for this loss. The gradient is torch's elementwise
    2 (pred - target) / n * grad, returned in pred's dtype."""

    @staticmethod
    def forward(ctx, pred: torch.Tensor, target: torch.Tensor):
        p = pred if pred.dtype in (torch.bfloat16, torch.float32) else pred.float()
        tg = target.float()
        if p.stride() != tg.stride() or not (p.is_contiguous() or p.is_contiguous(
                memory_format=torch.channels_last)):
            p, tg = p.contiguous(), tg.contiguous()
        n = p.numel()
        out = torch.empty((), device=p.device, dtype=torch.float32)
        ws_bytes = _lib.query("dpa_mse_loss_workspace_bytes")
        ws = torch.empty(ws_bytes, device=p.device, dtype=torch.uint8)
        dt = 1 if p.dtype == torch.float32 else 0  # DPA_DTYPE_F32 / DPA_DTYPE_BF16
        _lib.call("dpa_mse_loss_f32", p.data_ptr(), dt, tg.data_ptr(), n, out.data_ptr(),
                  ws.data_ptr(), ws_bytes, _lib.current_stream(p))
        ctx.save_for_backward(pred, target)
        return out

    @staticmethod
    def backward(ctx, grad):
        pred, target = ctx.saved_tensors
        d = (pred.float() - target.float()) * (2.0 / pred.numel())
        return (d * grad).to(pred.dtype), None


def mse_loss_hip(pred: torch.Tensor, target: torch.Tensor) -> torch.Tensor:
    """F.mse_loss(pred, target) on the GPU for operands of one shape. F.mse_loss broadcasts
    other shapes (with a warning); the kernel reads pred.numel() elements of each operand, so
    a mismatch is refused here rather than read out of bounds."""
    if pred.shape != target.shape:
        raise ValueError(f"mse_loss_hip: pred {tuple(pred.shape)} and target "
                         f"{tuple(target.shape)} differ in shape")
    if pred.device != target.device:
        raise ValueError(f"mse_loss_hip: pred on {pred.device}, target on {target.device}")
    return MSELossHIP.apply(pred, target)
