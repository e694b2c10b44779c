"""``python -m miracle_hip``: the command line (miracle_hip.cli)."""
import sys

from .cli import main

sys.exit(main())
