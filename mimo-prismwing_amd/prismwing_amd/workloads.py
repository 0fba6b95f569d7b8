"""Seeded synthetic workloads at the shapes of MiMo-V2.5's routed-MoE layer (hidden 4096, 256
experts of intermediate 2048, top-8, 128x128 f32 block scales), generated on the device.

Weights: per 128x128 block a scale log-uniform in [2^-10, 2^-6]; codes e4m3(clamp(N(0,1)/scale)).
Activations: N(0,1) rounded to bf16. Router: bf16 weights N(0, 0.02^2), f32 correction bias
U(-0.01, 0.01); the skewed variant adds kappa * (-s * ln rank_e) over a seeded permutation of expert
ranks (a Zipf(s) popularity profile injected through the bias).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List

import numpy as np

from .runtime import ExpertBank, Projection, WideMoeRuntime, route_from_logits

HIDDEN, INTERMEDIATE, EXPERTS, TOP_K = 4096, 2048, 256, 8
SEED_BASE = 0x50570000
ZIPF_S, ZIPF_KAPPA = 1.1, 0.05


def bf16_round_np(x: np.ndarray) -> np.ndarray:
    b = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000).astype(np.uint32).view(np.float32)


def bf16_bits_np(x: np.ndarray) -> np.ndarray:
    return (bf16_round_np(x).view(np.uint32) >> 16).astype(np.uint16)


@dataclass
class DeviceBank:
    """A layer's routed experts in HBM: gate/up [E, I, H], down [E, H, I] e4m3 + scale grids."""
    bank: ExpertBank
    gate_w: object
    up_w: object
    down_w: object
    gate_s: object
    up_s: object
    down_s: object
    projections: List[Projection] = field(default_factory=list)

    @property
    def weight_bytes_per_expert(self) -> int:
        E = self.gate_w.shape[0]
        return (self.gate_w.numel() + self.up_w.numel() + self.down_w.numel()) // E

    @property
    def scale_bytes_per_expert(self) -> int:
        E = self.gate_w.shape[0]
        return 4 * (self.gate_s.numel() + self.up_s.numel() + self.down_s.numel()) // E

    def expert_host(self, e: int):
        """(gate_w, gate_s, up_w, up_s, down_w, down_s) of expert e as numpy arrays."""
        return tuple(t[e].cpu().numpy() for t in (self.gate_w, self.gate_s, self.up_w, self.up_s,
                                                  self.down_w, self.down_s))


def synth_bank(rt: WideMoeRuntime, n_experts: int = EXPERTS, hidden: int = HIDDEN,
               inter: int = INTERMEDIATE, seed: int = SEED_BASE + 2) -> DeviceBank:
    import torch
    dev = torch.device("cuda", rt.device)
    gate_w = torch.empty((n_experts, inter, hidden), dtype=torch.uint8, device=dev)
    up_w = torch.empty_like(gate_w)
    down_w = torch.empty((n_experts, hidden, inter), dtype=torch.uint8, device=dev)
    gate_s = torch.empty((n_experts, inter // 128, hidden // 128), dtype=torch.float32, device=dev)
    up_s = torch.empty_like(gate_s)
    down_s = torch.empty((n_experts, hidden // 128, inter // 128), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    for i, (w, s, rows, cols) in enumerate(((gate_w, gate_s, n_experts * inter, hidden),
                                            (up_w, up_s, n_experts * inter, hidden),
                                            (down_w, down_s, n_experts * hidden, inter))):
        rt.synth_scales(s, s.numel(), seed * 16 + 2 * i)
        rt.synth_fp8(w, s, rows, cols, seed * 16 + 2 * i + 1)
    projs = []
    gates, ups, downs = [], [], []
    for e in range(n_experts):
        g = rt.bind_projection_device(gate_w[e], gate_s[e], inter, hidden)
        u = rt.bind_projection_device(up_w[e], up_s[e], inter, hidden)
        d = rt.bind_projection_device(down_w[e], down_s[e], hidden, inter)
        gates.append(g); ups.append(u); downs.append(d)
        projs += [g, u, d]
    bank = rt.expert_bank(gates, ups, downs)
    return DeviceBank(bank, gate_w, up_w, down_w, gate_s, up_s, down_s, projs)


def activations(rows: int, seed: int, hidden: int = HIDDEN) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return bf16_round_np(rng.standard_normal((rows, hidden)).astype(np.float32))


def router_inputs(seed: int, zipf: bool = False, experts: int = EXPERTS, hidden: int = HIDDEN):
    """(router weight as bf16-valued f32 [experts, hidden], bias f32 [experts])."""
    rng = np.random.default_rng(seed)
    w = bf16_round_np((rng.standard_normal((experts, hidden)) * 0.02).astype(np.float32))
    bias = rng.uniform(-0.01, 0.01, experts).astype(np.float32)
    if zipf:
        rank = rng.permutation(experts) + 1
        bias = (bias + ZIPF_KAPPA * (-ZIPF_S * np.log(rank))).astype(np.float32)
    return w, bias


def route_host(x: np.ndarray, router_w: np.ndarray, bias: np.ndarray):
    """Routes for a workload: f32 logits (numpy) -> the library's PyTorch-order routing."""
    logits = (x.astype(np.float32) @ router_w.T.astype(np.float32)).astype(np.float32)
    _, sel, w, ties = route_from_logits(logits, bias)
    return sel, w, ties


def unique_experts(sel: np.ndarray) -> int:
    return int(np.unique(sel).size)
