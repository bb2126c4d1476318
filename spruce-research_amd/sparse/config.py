"""Residual-summary settings shared by the command line and the attention call
(reference sparse/config.py:10-73).

``ResidualSummaryConfig`` carries the four ``residual_summaries`` /
``summary_*`` keyword arguments of ``sparse_prefill_attention_forward`` and
rejects what the attention call would reject: a prototype count outside
``SUMMARY_PROTOTYPES``, a mode outside ``SUMMARY_MODES``, and an enabled
learned mode without a checkpoint.  The argparse flags and their defaults are
the reference's, so its drivers parse the same command lines.
"""
from __future__ import annotations

from dataclasses import dataclass

SUMMARY_PROTOTYPES = (1, 2, 4)
SUMMARY_MODES = ("mean", "learned")

__all__ = ["SUMMARY_MODES", "SUMMARY_PROTOTYPES", "ResidualSummaryConfig",
           "add_residual_summary_arguments", "residual_summary_config_from_args"]


@dataclass(frozen=True)
class ResidualSummaryConfig:
    enabled: bool = False
    prototypes: int = 1
    mode: str = "mean"
    checkpoint: str | None = None

    def __post_init__(self) -> None:
        if self.prototypes not in SUMMARY_PROTOTYPES:
            raise ValueError(f"summary prototypes must be one of {SUMMARY_PROTOTYPES}, "
                             f"got {self.prototypes}")
        if self.mode not in SUMMARY_MODES:
            raise ValueError(f"summary mode must be one of {SUMMARY_MODES}, got {self.mode!r}")
        if self.enabled and self.mode == "learned" and not self.checkpoint:
            raise ValueError("learned summary mode requires --summary-checkpoint")

    def attention_kwargs(self) -> dict:
        """The keyword arguments of ``sparse_prefill_attention_forward`` this config sets."""
        return dict(residual_summaries=self.enabled, summary_prototypes=self.prototypes,
                    summary_mode=self.mode, summary_checkpoint=self.checkpoint)


_FLAGS = (
    ("--residual-summaries",
     dict(action="store_true",
          help="replace omitted causal blocks with deterministic tree-node K/V summaries")),
    ("--summary-prototypes",
     dict(type=int, choices=SUMMARY_PROTOTYPES, default=1,
          help="contiguous positional prototypes per residual tree node")),
    ("--summary-mode",
     dict(choices=SUMMARY_MODES, default="mean",
          help="summary compressor; learned mode requires a trained checkpoint")),
    ("--summary-checkpoint",
     dict(help="learned compressor checkpoint (unused by deterministic mean mode)")),
)


def add_residual_summary_arguments(parser) -> None:
    """Add the four residual-summary flags to an argparse parser."""
    for flag, options in _FLAGS:
        parser.add_argument(flag, **options)


def residual_summary_config_from_args(args) -> ResidualSummaryConfig:
    """The config a parsed namespace from ``add_residual_summary_arguments`` describes."""
    return ResidualSummaryConfig(enabled=bool(args.residual_summaries),
                                 prototypes=int(args.summary_prototypes),
                                 mode=str(args.summary_mode),
                                 checkpoint=args.summary_checkpoint)
