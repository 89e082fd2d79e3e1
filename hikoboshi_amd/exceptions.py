"""Structured errors of the Python API, one class per reference status code
(python/hikoboshi/exceptions.py; codes cpp/include/hikoboshi/universal/status.hpp:12-19)."""
from __future__ import annotations


class HikoboshiError(RuntimeError):
    """Base class; ``code`` is the snake_case status name, ``detail`` the message."""

    code = "internal_error"

    def __init__(self, detail: str = "", *, code: str | None = None) -> None:
        super().__init__(detail)
        self.detail = detail
        if code is not None:
            self.code = code
        self.status_code = self.code


class InvalidArgumentError(HikoboshiError):
    code = "invalid_argument"


class FailedPreconditionError(HikoboshiError):
    code = "failed_precondition"


class UnavailableError(HikoboshiError):
    code = "unavailable"


class UnimplementedError(HikoboshiError):
    code = "unimplemented"


class InternalError(HikoboshiError):
    code = "internal_error"


#: numeric StatusCode (the C ABI's hkbs_status) -> class
BY_STATUS = {1: InvalidArgumentError, 2: FailedPreconditionError, 3: UnavailableError, 4: UnimplementedError,
             5: InternalError}
#: CLI exit code per status (cpp/cli/exit_codes.cpp:28-42)
EXIT_CODES = {"invalid_argument": 2, "failed_precondition": 2, "unavailable": 3, "unimplemented": 4,
              "internal_error": 5}


def from_status(code: int, detail: str) -> HikoboshiError:
    return BY_STATUS.get(int(code), InternalError)(detail)


__all__ = ["HikoboshiError", "InvalidArgumentError", "FailedPreconditionError", "UnavailableError",
           "UnimplementedError", "InternalError", "from_status", "BY_STATUS", "EXIT_CODES"]
