"""Error types: the variants of ``PotError`` (src/error.rs:8-38 in the reference)
that the attention path can produce, keyed by the C ABI's status codes."""

BP_OK = 0
BP_ERR_CONFIG = -1
BP_ERR_CONTEXT_OVERFLOW = -2
BP_ERR_INVALID_ARG = -3
BP_ERR_HIP = -4
BP_ERR_DEVICE_LOST = -5
BP_ERR_OUT_OF_MEMORY = -6
BP_ERR_NO_DEVICE = -7


class PotError(Exception):
    """Base of every error raised by the binding (``PotError``)."""

    status = None

    def __init__(self, message, status=None):
        super().__init__(message)
        if status is not None:
            self.status = status


class ConfigError(PotError):
    """``PotError::Config``: invalid configuration or argument."""
    status = BP_ERR_CONFIG


class ContextOverflowError(PotError):
    """``PotError::ContextOverflow``: pos + tokens > max_seq."""
    status = BP_ERR_CONTEXT_OVERFLOW


class DeviceLostError(PotError):
    """``PotError::DeviceLost``: the model is permanently unusable; drop it,
    create a new one and restore a snapshot (src/model.rs:1719-1728)."""
    status = BP_ERR_DEVICE_LOST


class HipError(PotError):
    """A HIP runtime error that did not lose the device."""
    status = BP_ERR_HIP


class OutOfMemoryError(PotError):
    status = BP_ERR_OUT_OF_MEMORY


class NoAdapterError(PotError):
    """``PotError::NoAdapter``: no HIP device."""
    status = BP_ERR_NO_DEVICE


_BY_STATUS = {
    BP_ERR_CONFIG: ConfigError,
    BP_ERR_INVALID_ARG: ConfigError,
    BP_ERR_CONTEXT_OVERFLOW: ContextOverflowError,
    BP_ERR_HIP: HipError,
    BP_ERR_DEVICE_LOST: DeviceLostError,
    BP_ERR_OUT_OF_MEMORY: OutOfMemoryError,
    BP_ERR_NO_DEVICE: NoAdapterError,
}


def error_for(status: int, message: str) -> PotError:
    cls = _BY_STATUS.get(status, PotError)
    return cls(message, status)
