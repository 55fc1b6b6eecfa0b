"""MI355X-native zlib/DEFLATE codec; importing this package does not initialise the GPU.

Public API mirrors the reference package's exports (src/cuda_zlib/__init__.py:6-21).
"""

from ._codec import (compress_zlib, decompress_zlib, compile_kernels,
                     compress_zlib_padded, decompress_zlib_checked,
                     decompress_zlib_host, workspace_pool_stats, trim_workspace_pool)
from ._codec import (compress_zlib_batch_padded, decompress_zlib_batch_checked,
                     compress_zlib_batch, decompress_zlib_batch,
                     compress_zlib_batch_host, decompress_zlib_batch_host)
from ._codec import (decompress_gzip, decompress_gzip_checked, decompress_deflate_raw,
                     decompress_deflate_raw_checked)
from ._errors import BackendUnavailable, CodecError, UnsupportedStream

__all__ = ["compress_zlib", "decompress_zlib", "compile_kernels",
           "compress_zlib_padded", "decompress_zlib_checked", "decompress_zlib_host",
           "workspace_pool_stats", "trim_workspace_pool",
           "compress_zlib_batch_padded", "decompress_zlib_batch_checked",
           "compress_zlib_batch", "decompress_zlib_batch",
           "compress_zlib_batch_host", "decompress_zlib_batch_host",
           "decompress_gzip", "decompress_gzip_checked",
           "decompress_deflate_raw", "decompress_deflate_raw_checked",
           "BackendUnavailable", "CodecError", "UnsupportedStream"]
__version__ = "0.1.0"
