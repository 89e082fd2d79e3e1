"""Command line: ``python -m hikoboshi_amd design --pdb IN.pdb --out OUT.fasta [options]``.

Mirrors the reference's ``hikoboshi design`` (cpp/cli/commands/design.cpp): the
same options (``--opt VALUE`` or ``--opt=VALUE``), the same validation
messages, errors printed as ``hikoboshi: <status>: <detail>`` on stderr and the
exit codes of cpp/cli/exit_codes.cpp (2 invalid argument / failed
precondition, 3 unavailable, 4 unimplemented, 5 internal). Designs run on the
GPU through the same path as ``hikoboshi_amd.inverse_fold``.
"""
from __future__ import annotations

import ctypes
import sys

from .exceptions import EXIT_CODES, HikoboshiError, InvalidArgumentError

USAGE = ("usage: hikoboshi design --pdb INPUT.pdb --out OUT.fasta [options]\n"
         "\n"
         "options:\n"
         "  --num-seqs N             number of sequences to design (default 1)\n"
         "  --sampling-temp T        sampling temperature (default 0.1)\n"
         "  --seed N                 deterministic sampling seed (default 0)\n"
         "  --decode-order random|n_to_c\n"
         "  --package NAME           compiled ProteinMPNN package ID or alias\n"
         "  --backbone-noise SIGMA   coordinate noise sigma (default 0.0)\n"
         "  --out-logprobs PATH      write opt-in [N,L,21] log-prob NPZ\n")

#: historical or reserved flags the reference rejects (cpp/cli/options.cpp:76-83)
REJECTED = {"--soft", "--soft-sw", "--temperature", "--anneal", "--save-frames", "--tree", "--msa", "--database",
            "--gpu", "--simd"}

_libc = ctypes.CDLL(None)
_libc.strtof.restype = ctypes.c_float
_libc.strtof.argtypes = [ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p)]
_libc.strtoull.restype = ctypes.c_ulonglong
_libc.strtoull.argtypes = [ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p), ctypes.c_int]
_errno = ctypes.c_int.in_dll(_libc, "errno")


def _strto(fn, text: str, *extra):
    """C strtof / strtoull with the reference's full-consumption and errno checks."""
    raw = text.encode()
    buf = ctypes.create_string_buffer(raw)
    end = ctypes.c_char_p()
    _errno.value = 0
    value = fn(buf, ctypes.byref(end), *extra)
    consumed = ctypes.cast(end, ctypes.c_void_p).value - ctypes.addressof(buf)
    if _errno.value != 0 or consumed == 0 or consumed != len(raw):
        return None
    return value


def _option(args: list[str], i: int, name: str):
    """(matched, value or None, next index) for ``--name VALUE`` / ``--name=VALUE``."""
    arg = args[i]
    if arg == name:
        if i + 1 >= len(args):
            raise InvalidArgumentError("option requires a value")
        return True, args[i + 1], i + 1
    if len(arg) > len(name) + 1 and arg.startswith(name) and arg[len(name)] == "=":
        return True, arg[len(name) + 1:], i
    return False, None, i


def parse_design_options(args: list[str]) -> dict:
    opts = {"pdb": "", "out": "", "out_logprobs": "", "package": None, "sampling_temp": 0.1, "num_seqs": 1,
            "seed": 0, "decode_order": "random", "backbone_noise": 0.0}
    i = 0
    while i < len(args):
        arg = args[i]
        if arg in REJECTED:
            raise InvalidArgumentError("that historical or reserved flag is not available in Hikoboshi 0.1.0")
        matched, value, i = _option(args, i, "--package")
        if matched:
            from .inverse_fold import resolve_package
            resolve_package(value)
            opts["package"] = value
            i += 1
            continue
        for name in ("--external-package", "--package-path", "--weights"):
            if arg == name or arg.startswith(name + "="):
                raise InvalidArgumentError("external package paths are not supported in Hikoboshi 0.1.0; design "
                                           "uses the compiled ProteinMPNN registered package")
        handled = False
        for name, key in (("--pdb", "pdb"), ("--out", "out"), ("--out-logprobs", "out_logprobs")):
            matched, value, i = _option(args, i, name)
            if matched:
                opts[key] = value
                handled = True
                break
        if not handled:
            for name, key, parse, message in (
                    ("--sampling-temp", "sampling_temp", lambda v: _strto(_libc.strtof, v),
                     "sampling-temp must be a finite number"),
                    ("--backbone-noise", "backbone_noise", lambda v: _strto(_libc.strtof, v),
                     "backbone-noise must be a finite number"),
                    ("--num-seqs", "num_seqs", lambda v: _strto(_libc.strtoull, v, 10),
                     "num-seqs must be a positive integer"),
                    ("--seed", "seed", lambda v: _strto(_libc.strtoull, v, 10), "seed must be a non-negative integer")):
                matched, value, i = _option(args, i, name)
                if matched:
                    parsed = parse(value)
                    if parsed is None or (key == "num_seqs" and parsed == 0):
                        raise InvalidArgumentError(message)
                    opts[key] = parsed
                    handled = True
                    break
        if not handled:
            matched, value, i = _option(args, i, "--decode-order")
            if matched:
                if value not in ("random", "n_to_c", "n-to-c"):
                    raise InvalidArgumentError("decode-order must be random or n_to_c")
                opts["decode_order"] = "n_to_c" if value != "random" else "random"
                handled = True
        if not handled:
            if arg.startswith("-"):
                raise InvalidArgumentError("unknown design option")
            raise InvalidArgumentError("design requires explicit --pdb and --out options")
        i += 1
    if not opts["pdb"]:
        raise InvalidArgumentError("design requires --pdb")
    if not opts["out"]:
        raise InvalidArgumentError("design requires --out")
    return opts


def run_design(args: list[str]) -> int:
    if args and args[0] in ("-h", "--help"):
        sys.stdout.write(USAGE)
        return 0
    from . import design_io
    from .inverse_fold import design, load_structure

    opts = parse_design_options(args)
    bb, native = load_structure(opts["pdb"])
    result = design(bb, native, num_seqs=int(opts["num_seqs"]), sampling_temp=opts["sampling_temp"],
                    seed=int(opts["seed"]), decode_order=opts["decode_order"], backbone_noise=opts["backbone_noise"])
    design_io.write_design_fasta(opts["out"], result.sequences, opts["sampling_temp"])
    if opts["out_logprobs"]:
        design_io.write_inverse_fold_logprobs_npz(opts["out_logprobs"], result.log_prob_values)
    return 0


def main(argv: list[str] | None = None) -> int:
    argv = sys.argv[1:] if argv is None else argv
    if not argv or argv[0] in ("-h", "--help"):
        sys.stdout.write(USAGE)
        return 0 if argv else 2
    command, rest = argv[0], argv[1:]
    try:
        if command == "design":
            return run_design(rest)
        raise InvalidArgumentError(f"unknown command: {command} (this build provides: design)")
    except HikoboshiError as exc:
        detail = f": {exc.detail}" if exc.detail else ""
        sys.stderr.write(f"hikoboshi: {exc.code}{detail}\n")
        return EXIT_CODES.get(exc.code, 5)


if __name__ == "__main__":
    sys.exit(main())
