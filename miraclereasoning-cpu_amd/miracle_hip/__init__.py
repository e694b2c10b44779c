"""MI355X-native per-token forward path for the Miracle model families."""
from .config import ModelConfig

__all__ = ["ModelConfig"]
