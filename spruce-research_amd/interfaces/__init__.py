"""The frozen selected_blocks interface (interfaces/selected_blocks_spec.md)."""
from pkgutil import extend_path

__path__ = extend_path(__path__, __name__)

from interfaces.validator import LOCAL_WINDOW, PAD_VALUE, validate_selected_blocks

__all__ = ["LOCAL_WINDOW", "PAD_VALUE", "validate_selected_blocks"]
