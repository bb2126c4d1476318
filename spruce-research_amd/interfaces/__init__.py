"""The frozen selected_blocks interface (interfaces/selected_blocks_spec.md)."""
from interfaces.validator import LOCAL_WINDOW, PAD_VALUE, validate_selected_blocks

__all__ = ["LOCAL_WINDOW", "PAD_VALUE", "validate_selected_blocks"]
