"""Stand-alone kernels behind boonta's network blocks (boonta/networks/kernels)."""
from .scan import get_scan_implementation, hip, scan

__all__ = ["get_scan_implementation", "hip", "scan"]
