"""Stand-alone kernels behind boonta's network blocks (boonta/networks/kernels)."""
from .scan import get_scan_implementation, hip, scan, ssm, ssm_scan

__all__ = ["get_scan_implementation", "hip", "scan", "ssm", "ssm_scan"]
