"""MI355X-native paged-KV hot path (slot-mapped append, block-table GQA decode,
split-K decode) with the reference's Python API and KV-pool structures."""

__all__ = ["kernels"]
