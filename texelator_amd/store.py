"""State directory (``texelator/store.py:10-15`` of the reference) and name sanitising."""
from __future__ import annotations

import os
import re
from pathlib import Path

_default_state = Path.home() / ".cache" / "texelator_amd"
STATE_HOME = Path(os.environ.get("TEXELATOR_HOME", _default_state)).expanduser().resolve()


def safe_name(value: str) -> str:
    """``texelator/store.py:32-33``."""
    return re.sub(r"[^A-Za-z0-9_.-]+", "-", value).strip("-").lower()
