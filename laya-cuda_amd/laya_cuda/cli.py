"""Command line: `python -m laya_cuda predict|doctor` (the reference's laya-cuda CLI,
laya_cuda/cli.py:179-215, for the commands that need no network: `models` and `download` list and
fetch hosted checkpoints, which this runtime does not do).

  predict STATE -q QUESTIONS [-m MODEL]     one answer dict as JSON
  predict -i REQUESTS.jsonl [-q QUESTIONS]  one JSON line per request line {"id", "state",
                                            "questions"}; a failing line gets an "error" field and
                                            the exit status becomes 1, the other lines still run
  doctor [MODEL] [--json]                   library, devices, a seeded forward, optionally a model

QUESTIONS is inline JSON, a file, or - (stdin).  Native code loads only inside the commands.
"""
import argparse
import json
import sys
from pathlib import Path

from . import __version__


class UsageError(Exception):
    """A mistake in the command line or its inputs, reported in one line."""


def _json_arg(value, what):
    text = value
    if value == "-":
        text = sys.stdin.read()
    elif not value.lstrip().startswith(("{", "[")):
        try:
            text = Path(value).read_text(encoding="utf-8")
        except OSError as error:
            raise UsageError(f"cannot read {what} {value!r}: {error.strerror}") from None
    try:
        return json.loads(text)
    except json.JSONDecodeError as error:
        raise UsageError(f"{what} are not valid JSON: {error}") from None


def _emit(stream, value, pretty=False):
    stream.write(json.dumps(value, ensure_ascii=False, indent=2 if pretty else None, default=str) + "\n")


def cmd_predict(args):
    from .engine import Engine
    if (args.state is None) == (args.input is None):
        raise UsageError("give exactly one of STATE or --input")
    shared = _json_arg(args.questions, "questions") if args.questions else None
    out = open(args.output, "w", encoding="utf-8") if args.output else sys.stdout
    failed = 0
    try:
        with Engine(args.model, device=args.device) as engine:
            if args.state is not None:
                if shared is None:
                    raise UsageError("--questions is required with a STATE")
                state = sys.stdin.read() if args.state == "-" else args.state
                answer = engine.predict(state, shared)
                if args.metrics:
                    answer["metrics"] = engine.last_metrics
                _emit(out, answer, pretty=out is sys.stdout)
                return 0
            lines = sys.stdin if args.input == "-" else open(args.input, encoding="utf-8")
            with lines:
                for number, line in enumerate(lines, 1):
                    if not line.strip():
                        continue
                    record = {"id": number}
                    try:
                        request = json.loads(line)
                        if not isinstance(request, dict) or "state" not in request:
                            raise ValueError('each line must be an object with a "state"')
                        record["id"] = request.get("id", number)
                        questions = request.get("questions", shared)
                        if questions is None:
                            raise ValueError('no "questions" on the line and no --questions')
                        record.update(engine.predict(request["state"], questions))
                        if args.metrics:
                            record["metrics"] = engine.last_metrics
                    except Exception as error:  # a bad line fails alone
                        failed += 1
                        record["error"] = f"{type(error).__name__}: {error}"
                    _emit(out, record)
                    out.flush()
    finally:
        if out is not sys.stdout:
            out.close()
    if failed:
        print(f"laya: {failed} request(s) failed (see their \"error\" field)", file=sys.stderr)
    return 1 if failed else 0


def cmd_doctor(args):
    from . import doctor
    if not args.json:
        print(doctor.header(), flush=True)
    report = doctor.run(args.model, args.device, echo=None if args.json else lambda line: print(line, flush=True))
    if args.json:
        _emit(sys.stdout, {"version": __version__, "header": doctor.header(), "passed": report.passed,
                           "checks": report.checks}, pretty=True)
    else:
        print("All checks passed." if report.passed else "Some checks failed.")
    return 0 if report.passed else 1


def parser():
    p = argparse.ArgumentParser(prog="python -m laya_cuda", description="Laya decision models on MI355X (HIP).")
    p.add_argument("--version", action="version", version=f"laya-mi355x {__version__}")
    sub = p.add_subparsers(dest="command", required=True, metavar="COMMAND")
    pr = sub.add_parser("predict", help="answer questions about a state")
    pr.add_argument("state", nargs="?", help="state text, or - for stdin")
    pr.add_argument("-q", "--questions", help="questions: inline JSON, a file, or -")
    pr.add_argument("-i", "--input", help="JSONL requests, one per line (- for stdin)")
    pr.add_argument("-o", "--output", help="write to this file instead of stdout")
    pr.add_argument("-m", "--model", default="laya", help="checkpoint directory or registry alias")
    pr.add_argument("--device", default="cuda:0")
    pr.add_argument("--metrics", action="store_true", help="include timing metrics")
    pr.set_defaults(run=cmd_predict)
    dr = sub.add_parser("doctor", help="check the library, the HIP devices and a forward")
    dr.add_argument("model", nargs="?", help="also load this checkpoint and time predictions")
    dr.add_argument("--device", default="cuda:0")
    dr.add_argument("--json", action="store_true", help="machine-readable report")
    dr.set_defaults(run=cmd_doctor)
    return p


def main(argv=None):
    args = parser().parse_args(argv)
    try:
        return args.run(args)
    except UsageError as error:
        print(f"laya: {error}", file=sys.stderr)
        return 2
    except (ValueError, FileNotFoundError, RuntimeError) as error:
        print(f"laya: {type(error).__name__}: {error}", file=sys.stderr)
        return 1
