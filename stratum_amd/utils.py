"""Structured event logging (``stratum/utils.py:25-42``)."""

from __future__ import annotations

import logging

_log = logging.getLogger("stratum_amd")


def log_event(event: str, **fields) -> None:
    """Log ``[stratum] <event> k=v ...`` at INFO."""
    parts = " ".join(f"{k}={v}" for k, v in fields.items())
    _log.info("[stratum] %s %s", event, parts)
