"""Attention error metrics and the numerical gate.

The metric set (finite, max_abs, mean_abs, relative L2, cosine, optional
selected/possible block counts) and the gate semantics follow the reference's
``turing_sage/correctness.py:16-94``.  Never imported by the attention hot path.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class AttentionCorrectnessResult:
    candidate: str
    reference: str
    shape: tuple
    dtype: torch.dtype
    finite: bool
    max_abs: float
    mean_abs: float
    relative_l2: float
    cosine: float
    selected_blocks: int | None = None
    possible_blocks: int | None = None


def attention_error_metrics(
    candidate: torch.Tensor,
    reference: torch.Tensor,
    *,
    candidate_name: str = "candidate",
    reference_name: str = "reference",
    selected_blocks: int | None = None,
    possible_blocks: int | None = None,
) -> AttentionCorrectnessResult:
    """Metrics in float64; a shape mismatch raises before any reduction."""
    if candidate.shape != reference.shape:
        raise AssertionError(
            f"{candidate_name} shape {tuple(candidate.shape)} != {reference_name} shape {tuple(reference.shape)}"
        )
    a = candidate.detach().double().flatten()
    b = reference.detach().double().flatten()
    diff = a - b
    b_norm = torch.linalg.vector_norm(b)
    a_norm = torch.linalg.vector_norm(a)
    return AttentionCorrectnessResult(
        candidate=candidate_name,
        reference=reference_name,
        shape=tuple(candidate.shape),
        dtype=candidate.dtype,
        finite=bool(torch.isfinite(a).all().item()),
        max_abs=float(diff.abs().max().item()) if diff.numel() else 0.0,
        mean_abs=float(diff.abs().mean().item()) if diff.numel() else 0.0,
        relative_l2=float((torch.linalg.vector_norm(diff) / b_norm.clamp_min(1e-12)).item()),
        cosine=float((torch.dot(a, b) / (a_norm * b_norm).clamp_min(1e-12)).item()),
        selected_blocks=selected_blocks,
        possible_blocks=possible_blocks,
    )


def require_attention_correctness(
    result: AttentionCorrectnessResult,
    *,
    max_abs: float,
    cosine: float,
    relative_l2: float | None = None,
) -> None:
    """Raises AssertionError listing every bound the result fails."""
    problems = []
    if not result.finite:
        problems.append("non-finite output")
    if result.max_abs > max_abs:
        problems.append(f"max_abs={result.max_abs:.6g}>{max_abs:.6g}")
    if relative_l2 is not None and result.relative_l2 > relative_l2:
        problems.append(f"relative_l2={result.relative_l2:.6g}>{relative_l2:.6g}")
    if result.cosine < cosine:
        problems.append(f"cosine={result.cosine:.6g}<{cosine:.6g}")
    if result.possible_blocks is not None and result.selected_blocks != result.possible_blocks:
        problems.append(f"dense route selected {result.selected_blocks}/{result.possible_blocks} blocks")
    if problems:
        raise AssertionError(
            f"{result.candidate} vs {result.reference} failed the attention gate: " + "; ".join(problems)
        )
