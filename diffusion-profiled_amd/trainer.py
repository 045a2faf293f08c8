"""Graph-captured single-GPU training step (train.py:104-149 of the reference).

``prepare_cuda_graph`` keeps the reference's signature and order: three warm-up iterations on
a side stream (which also lets every FP8 op and library kernel initialise outside the
capture), then one capture of zero_grad / autocast forward / loss accumulation / backward /
clip_grad_norm_ / AdamW / EMA. Replaying the returned graph is one training step. Every FP8
launch goes to torch's current stream, which is the capture stream inside the graph, and all
of their buffers come from torch's allocator (the graph's private pool).

``TrainState`` bundles model, optimizer, diffusion wrapper, EMA and the static input buffers
so a benchmark or test can build the reference's training setup in one call.

``save_checkpoint`` / ``load_checkpoint`` use the reference's file format (train.py:85-91).
"""
from __future__ import annotations

import dataclasses
import os

import torch

from .ddpm import DiffusionWrapper, EWMAWrapper
from .optim import FusedAdamWEMA
from .unet import UNet, UNetConfig


CHECKPOINT_KEYS = ("model_state_dict", "step", "config")
_COMPILED_PREFIX = "_orig_mod."  # state_dict prefix of a torch.compile'd module


def save_checkpoint(model: torch.nn.Module, step: int, config: dict, filename: str) -> None:
    """train.py:85-91: ``{"model_state_dict": model.state_dict(), "step": step, "config":
    config}`` written with torch.save. The reference passes its EMA model and
    ``UNetConfig.as_dict()`` plus ``hparams.*`` entries; the keys of this build's state dict
    are the reference's (module tree, parameter and FP8 window buffer names)."""
    torch.save({"model_state_dict": model.state_dict(), "step": int(step), "config": config},
               filename)


def config_from_dict(config: dict) -> UNetConfig:
    """The UNetConfig of a checkpoint's ``config``: the dataclass fields it names (the
    reference's ``hparams.*`` and any other keys are not model fields and are skipped)."""
    names = {f.name for f in dataclasses.fields(UNetConfig)}
    return UNetConfig(**{k: v for k, v in config.items() if k in names})


def load_checkpoint(filename: str | os.PathLike, model: torch.nn.Module | None = None,
                    map_location="cpu", strict: bool = True):
    """Reads a checkpoint in the reference's format with ``torch.load(weights_only=True)``
    (tensors, numbers, strings and containers only; nothing in the file is executed).
    State dicts saved from a torch.compile'd module (the reference compiles its model and
    its EMA copy, train.py:251, diffusion/ddpm.py:16) carry an ``_orig_mod.`` prefix, which
    is removed. Loads into ``model`` (built from the checkpoint's config when None) and
    returns ``(model, step, config)``."""
    ck = torch.load(filename, map_location=map_location, weights_only=True)
    if not isinstance(ck, dict) or any(k not in ck for k in CHECKPOINT_KEYS):
        raise KeyError(f"{filename}: not a checkpoint with keys {CHECKPOINT_KEYS}")
    sd = {(k[len(_COMPILED_PREFIX):] if k.startswith(_COMPILED_PREFIX) else k): v
          for k, v in ck["model_state_dict"].items()}
    config = ck["config"]
    if model is None:
        model = UNet(config_from_dict(config))
    model.load_state_dict(sd, strict=strict)
    return model, int(ck["step"]), config


def _one_step(ddpm: DiffusionWrapper, model: torch.nn.Module, ema_ddpm: DiffusionWrapper,
              static_batch: torch.Tensor, optimizer: torch.optim.Optimizer,
              loss_acc: torch.Tensor | None, static_t: torch.Tensor | None,
              static_eps: torch.Tensor | None, max_norm: float) -> torch.Tensor:
    optimizer.zero_grad(set_to_none=True)
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        loss = ddpm.forward_batch(static_batch, static_t, static_eps)
    if loss_acc is not None:
        loss_acc.add_(loss.detach())
    loss.backward()
    if getattr(optimizer, "fuses_clip_and_ema", False):
        optimizer.step()       # clip_grad_norm_ + AdamW + EMA in one pass (optim.FusedAdamWEMA)
    else:
        torch.nn.utils.clip_grad_norm_(model.parameters(), max_norm=max_norm)
        optimizer.step()
        ema_ddpm.model.update(ddpm.model)
    return loss


def prepare_cuda_graph(ddpm: DiffusionWrapper, model: torch.nn.Module, ema_ddpm: DiffusionWrapper,
                       static_batch: torch.Tensor, optimizer: torch.optim.Optimizer,
                       loss_acc: torch.Tensor, static_t: torch.Tensor | None = None,
                       static_eps: torch.Tensor | None = None, warmup: int = 3,
                       max_norm: float = 1.0) -> torch.cuda.CUDAGraph:
    """train.py:104-149. ``static_t`` / ``static_eps`` (optional) fix the timesteps and noise
    instead of drawing them inside the graph."""
    model.train()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(warmup):
            _one_step(ddpm, model, ema_ddpm, static_batch, optimizer, None, static_t, static_eps,
                      max_norm)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()

    g = torch.cuda.CUDAGraph()
    optimizer.zero_grad(set_to_none=True)
    with torch.cuda.graph(g):
        _one_step(ddpm, model, ema_ddpm, static_batch, optimizer, loss_acc, static_t, static_eps,
                  max_norm)
    return g


class TrainState:
    """Model + AdamW + DDPM + EMA with static input buffers (the reference's train.py setup:
    channels-last model, fused capturable AdamW, EMA beta 0.9999)."""

    def __init__(self, config: UNetConfig, batch: int, lr: float = 2e-4, max_t: int = 1000,
                 schedule_type: str = "linear", ema_beta: float = 0.9999, device: str = "cuda",
                 seed: int = 0, fixed_noise: bool = False, fused_tail: bool = True):
        torch.manual_seed(seed)
        model = UNet(config).to(memory_format=torch.channels_last)
        self.model = model.to(device)
        self.optimizer = torch.optim.AdamW(self.model.parameters(), lr=lr, fused=True,
                                           capturable=True)
        self.ddpm = DiffusionWrapper(self.model, schedule_type=schedule_type, max_t=max_t,
                                     in_dim=config.in_resolution, device=device)
        self.ema_ddpm = DiffusionWrapper(EWMAWrapper(self.model, beta=ema_beta),
                                         schedule_type=schedule_type, max_t=max_t,
                                         in_dim=config.in_resolution, device=device)
        # after the EMA copy: only the trained model prepares its FP8 weights per step
        on_gpu = device == "cuda" or str(device).startswith("cuda")
        self.model.weight_prep_enabled = on_gpu
        if on_gpu and fused_tail:
            # clip_grad_norm_(1.0) + AdamW (torch defaults) + EMA(ema_beta) in one fused pass
            self.optimizer = FusedAdamWEMA(self.model, self.ema_ddpm.model.model, lr=lr,
                                           max_norm=1.0, ema_beta=ema_beta)
        shape = (batch, config.in_channels, config.in_resolution, config.in_resolution)
        self.static_batch = torch.empty(shape, device=device).contiguous(
            memory_format=torch.channels_last)
        self.static_t = torch.zeros(batch, dtype=torch.long, device=device) if fixed_noise else None
        self.static_eps = (torch.zeros(shape, device=device).contiguous(
            memory_format=torch.channels_last) if fixed_noise else None)
        self.loss_acc = torch.zeros((), device=device)
        self.graph: torch.cuda.CUDAGraph | None = None

    def set_batch(self, images: torch.Tensor, t: torch.Tensor | None = None,
                  eps: torch.Tensor | None = None) -> None:
        self.static_batch.copy_(images)
        if t is not None:
            assert self.static_t is not None
            self.static_t.copy_(t)
        if eps is not None:
            assert self.static_eps is not None
            self.static_eps.copy_(eps)

    def eager_step(self) -> torch.Tensor:
        self.model.train()
        return _one_step(self.ddpm, self.model, self.ema_ddpm, self.static_batch, self.optimizer,
                         self.loss_acc, self.static_t, self.static_eps, 1.0)

    def capture(self, warmup: int = 3) -> torch.cuda.CUDAGraph:
        self.graph = prepare_cuda_graph(self.ddpm, self.model, self.ema_ddpm, self.static_batch,
                                        self.optimizer, self.loss_acc, self.static_t,
                                        self.static_eps, warmup=warmup)
        return self.graph

    def replay(self) -> None:
        assert self.graph is not None, "capture() first"
        self.graph.replay()
