"""A dated conformance record of the integer forward on this machine.

    python -m eii.conformance VECROOT [--record-dir DIR] [--sets t24,t128,t160]
                              [--cpu-checker PROG] [--variant FLAGS ...] [--no-variants]

The steps of tools/record_conformance.sh:17-84, on an MI355X:

* environment: date, host, commit and tree state, gcc, hipcc, the device eii_check reports,
  python;
* vector hashes: VECROOT/vectors.sha256 verified (tools/hash_vectors.sh --check);
* CPU check (optional): PROG SET VECROOT for every set, PROG being any checker with the
  `prog VECTORDIR [MODELDIR]` command line, e.g. the reference's scalar C checker c/intref.c
  (the reference's `make -C c check`);
* GPU check: eii_check SET on every set, and the count of ALL STATES EXACT lines;
* negative test: a copy of the first set with +1 on the aligned int32 in the middle of
  exp_resid_out.i32 (record_conformance.sh:44-63) must be reported with exit status 1 and a
  DIFFERS or MISMATCH line;
* build variants: libeii.so and eii_check rebuilt from the sources with other optimization
  flags, each exact on every set (record_conformance.sh:65-78).  Defaults:
  "-O3 -Xarch_host -O0": the host code (engine, C ABI, checker) unoptimized and the device code
  optimized, which is what the reference's "nvcc -O0" variant builds (nvcc's -O sets the host
  compiler's level; the device assembler keeps its default optimization); "-O1" and
  "-O2 -ffp-contract=off" for host and device code alike.  Device code cannot be built at -O0:
  the LDS DMA and scalar-register operands of the GEMM need values the compiler proves
  uniform, which it does only when optimizing.

Everything is printed and appended to DIR/run-YYYYmmdd-HHMMSS.txt (default DIR:
./conformance_runs); the last lines are RECORD OK or RECORD HAS FAILURES and the record's path.
Exit status 0 when every step passed, 1 otherwise.  The tool itself never touches the GPU:
every device step is an eii_check process.
"""
import argparse
import datetime
import os
import platform
import re
import shlex
import shutil
import subprocess
import sys
import tempfile

from .export_vectors import hash_root

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CHECKER = os.path.join(PKG, "eii_check")
DEFAULT_VARIANTS = ("-O3 -Xarch_host -O0", "-O1", "-O2 -ffp-contract=off")
DEFAULT_SETS = ("t24", "t128", "t160")
EXACT = "ALL STATES EXACT"


def plant_one_unit(path):
    """Add 1 to the aligned int32 in the middle of the file at path (little-endian, in place);
    returns its byte offset (tools/record_conformance.sh:46-54)."""
    with open(path, "r+b") as f:
        b = bytearray(f.read())
        i = len(b) // 2 // 4 * 4
        v = int.from_bytes(b[i:i + 4], "little", signed=True) + 1
        f.seek(i)
        f.write(v.to_bytes(4, "little", signed=True))
    return i


def _first_line(cmd):
    try:
        r = subprocess.run(cmd, capture_output=True, text=True, timeout=60)
        lines = (r.stdout or r.stderr).strip().splitlines()
        return lines[0] if lines else "(no output)"
    except (OSError, subprocess.SubprocessError) as e:
        return f"(unavailable: {e.__class__.__name__})"


def _git(*args):
    try:
        r = subprocess.run(["git", "-C", PKG] + list(args), capture_output=True, text=True, timeout=60)
        return r.stdout.strip() if r.returncode == 0 else None
    except (OSError, subprocess.SubprocessError):
        return None


class Record:
    def __init__(self, path):
        self.path = path
        self.f = open(path, "w")
        self.ok = True
        self.stopped = False   # a checker hung, crashed or reported a device error

    def say(self, text=""):
        print(text, flush=True)
        self.f.write(text + "\n")
        self.f.flush()

    def section(self, name):
        self.say("")
        self.say(f"== {name} ==")

    def log(self, text):
        """Tool output: into the record only (the reference appends make's output there)."""
        self.f.write(text if text.endswith("\n") or not text else text + "\n")
        self.f.flush()

    def fail(self, text):
        self.ok = False
        self.say(text)


def _run_checker(rec, prog, vecdir, modeldir, timeout, device=True):
    cmd = [prog, vecdir] + ([modeldir] if modeldir else [])
    rec.log("$ " + " ".join(shlex.quote(c) for c in cmd))
    try:
        r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout)
    except subprocess.TimeoutExpired:
        rec.log(f"(killed after {timeout} s)")
        rec.stopped = rec.stopped or device
        return None, ""
    rec.log(r.stdout + r.stderr)
    if device and (r.returncode < 0 or r.returncode == 3):
        # killed by a signal, or a device error: no further device step is started
        rec.stopped = True
    return r.returncode, r.stdout


def _model_dir(root, name):
    d = os.path.join(root, name)
    return d if os.path.exists(os.path.join(d, "model.bin")) else root


def record(vecroot, record_dir="conformance_runs", sets=DEFAULT_SETS, cpu_checker=None,
           variants=DEFAULT_VARIANTS, checker=CHECKER, timeout=900):
    """Run every step; returns (status, record path)."""
    vecroot = os.path.abspath(vecroot)
    os.makedirs(record_dir, exist_ok=True)
    stamp = datetime.datetime.now().strftime("%Y%m%d-%H%M%S")
    rec = Record(os.path.join(record_dir, f"run-{stamp}.txt"))
    sets = [s for s in sets if os.path.isdir(os.path.join(vecroot, s))]

    rec.section("environment")
    rec.say(f"date: {datetime.datetime.now(datetime.timezone.utc).strftime('%Y-%m-%dT%H:%M:%SZ')}")
    u = platform.uname()
    rec.say(f"host: {u.system} {u.release} {u.machine}")
    head = _git("rev-parse", "HEAD")
    if head:
        rec.say(f"commit: {head}")
        rec.say(f"tree: {'dirty' if _git('status', '--porcelain') else 'clean'}")
    rec.say(f"gcc: {_first_line(['gcc', '--version'])}")
    rec.say(f"hipcc: {_first_line([os.environ.get('HIPCC', '/opt/rocm/bin/hipcc'), '--version'])}")
    rec.say(f"python: {platform.python_version()}")
    rec.say(f"sets: {' '.join(sets) if sets else '(none found)'}")
    if not sets:
        rec.fail(f"no vector set of {', '.join(DEFAULT_SETS)} under {vecroot}")

    rec.section("vector hashes")
    if os.path.exists(os.path.join(vecroot, "vectors.sha256")):
        if hash_root(vecroot, check=True) == 0:
            rec.say("vectors match vectors.sha256")
        else:
            rec.fail("VECTOR HASH MISMATCH")
    else:
        rec.fail(f"no vectors.sha256 in {vecroot}")

    rec.section("CPU check")
    n_expected = 0
    if cpu_checker:
        ok = True
        for s in sets:
            rc, out = _run_checker(rec, cpu_checker, os.path.join(vecroot, s), _model_dir(vecroot, s), timeout,
                                   device=False)
            ok = ok and rc == 0 and EXACT in out
            n_expected += 1
        rec.say(f"cpu [{cpu_checker}]: pass" if ok else f"cpu [{cpu_checker}]: FAIL")
        rec.ok = rec.ok and ok
    else:
        rec.say("cpu: skipped (no --cpu-checker given)")

    rec.section("GPU check (eii_check)")
    ok = True
    device = None
    for s in sets:
        if rec.stopped:
            ok = False
            break
        rc, out = _run_checker(rec, checker, os.path.join(vecroot, s), _model_dir(vecroot, s), timeout)
        ok = ok and rc == 0 and EXACT in out
        n_expected += 1
        m = re.search(r"^device: (.*)$", out, re.M)
        device = device or (m.group(1) if m else None)
    if device:
        rec.say(f"gpu: {device}")
    rec.say("eii_check: pass" if ok else "eii_check: FAIL")
    rec.ok = rec.ok and ok
    with open(rec.path) as f:
        n_exact = sum(1 for line in f if EXACT in line and not line.startswith("exact lines"))
    rec.say(f"exact lines: {n_exact} ({n_expected} expected, one per set and checker)")
    if n_exact != n_expected:
        rec.ok = False

    tmp = tempfile.mkdtemp(prefix="eii_conformance_")
    try:
        rec.section("negative test (one unit changed in the expected states)")
        if rec.stopped:
            rec.fail("negative test: not run (a device step failed above)")
        elif sets:
            s = sets[0]
            src = os.path.join(vecroot, s)
            bad = os.path.join(tmp, s + "_bad")
            os.makedirs(bad)
            for name in os.listdir(src):
                p = os.path.join(src, name)
                if name == "exp_resid_out.i32":
                    shutil.copyfile(p, os.path.join(bad, name))
                elif not os.path.isdir(p):
                    os.symlink(os.path.realpath(p), os.path.join(bad, name))
            off = plant_one_unit(os.path.join(bad, "exp_resid_out.i32"))
            rec.say(f"{s}/exp_resid_out.i32: +1 at byte {off}")
            rc, out = _run_checker(rec, checker, bad, _model_dir(vecroot, s), timeout)
            hits = [l for l in out.splitlines() if re.search("DIFFERS|MISMATCH", l)]
            if rc == 1 and hits:
                rec.say("negative test: detected")
                for l in hits[:3]:
                    rec.say(l)
            else:
                rec.fail(f"negative test: NOT DETECTED (exit {rc}; the check cannot fail, investigate)")

        rec.section("build variants")
        for flags in variants:
            if rec.stopped:
                rec.fail(f"variant [{flags}]: not run (a device step failed above)")
                continue
            out_dir = os.path.join(tmp, "variant")
            shutil.rmtree(out_dir, ignore_errors=True)
            cmd = [sys.executable, os.path.join(PKG, "build.py"), "--out", out_dir, "--opt=" + flags]
            rec.log("$ " + " ".join(shlex.quote(c) for c in cmd))
            b = subprocess.run(cmd, capture_output=True, text=True)
            rec.log(b.stdout + b.stderr)
            if b.returncode != 0:
                rec.fail(f"variant [{flags}]: build failed")
                continue
            ok = bool(sets)
            for s in sets:
                if rec.stopped:
                    ok = False
                    break
                rc, out = _run_checker(rec, os.path.join(out_dir, "eii_check"), os.path.join(vecroot, s),
                                       _model_dir(vecroot, s), timeout)
                ok = ok and rc == 0 and EXACT in out
            if ok:
                rec.say(f"variant [{flags}]: exact on {' '.join(sets)}")
            else:
                rec.fail(f"variant [{flags}]: FAIL")
        if not variants:
            rec.say("variants: skipped")
    finally:
        shutil.rmtree(tmp, ignore_errors=True)

    rec.section("result")
    rec.say("RECORD OK" if rec.ok else "RECORD HAS FAILURES")
    rec.say(f"written to {rec.path}")
    rec.f.close()
    return (0 if rec.ok else 1), rec.path


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("vecroot", help="directory holding model.bin, vectors.sha256 and the vector sets")
    ap.add_argument("--record-dir", default="conformance_runs")
    ap.add_argument("--sets", default=",".join(DEFAULT_SETS), help="comma-separated set directories")
    ap.add_argument("--cpu-checker", help="a CPU checker with the `prog VECTORDIR [MODELDIR]` command line")
    ap.add_argument("--variant", action="append", help="optimization flags of a build variant (repeatable)")
    ap.add_argument("--no-variants", action="store_true")
    ap.add_argument("--timeout", type=int, default=900, help="seconds per checker run")
    a = ap.parse_args(argv)
    variants = () if a.no_variants else tuple(a.variant or DEFAULT_VARIANTS)
    status, _ = record(a.vecroot, a.record_dir, a.sets.split(","), a.cpu_checker, variants, timeout=a.timeout)
    return status


if __name__ == "__main__":
    sys.exit(main())
