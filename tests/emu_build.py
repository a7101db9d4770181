"""Builds the CPU wavefront-emulator drivers of tests/wave_emu (test
infrastructure): the library's HIP sources are copied and rewritten for the
emulator (tests/wave_emu/prep.py), then compiled with the host clang++, one
object per source and define set, in parallel."""
import concurrent.futures
import os
import shutil
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CXX = "/opt/rocm/llvm/bin/clang++"


def available() -> bool:
    return os.path.exists(CXX) or shutil.which(CXX) is not None


_shared = {}  # per process: the rewritten sources and every library object built so far


def _library_tree():
    """The library sources rewritten for the emulator, once per process."""
    if "src" not in _shared:
        import atexit
        import tempfile
        top = tempfile.mkdtemp(prefix="tau_emu_")
        atexit.register(shutil.rmtree, top, True)
        src = os.path.join(top, "src")
        sys.path.insert(0, os.path.join(ROOT, "tests", "wave_emu"))
        import prep
        prep.main(ROOT, src)
        _shared["src"] = src
        _shared["objects"] = {}
    return _shared["src"]


def build(out_dir, driver: str, variants):
    """variants: {name: (sources, defines)}; returns {name: binary path}.
    Library objects are compiled once per process and shared by every driver."""
    out_dir = str(out_dir)
    src = _library_tree()
    objects = _shared["objects"]
    csrc = os.path.join(src, "a", "csrc")
    inc = ["-I", os.path.join(ROOT, "tests", "wave_emu"), "-I", csrc]
    flags = ["-std=c++20", "-O1", "-w"]
    jobs = {}  # (file, defines) -> object still to compile
    drv = os.path.join(ROOT, "tests", "wave_emu", driver)
    for sources, defines in variants.values():
        for f in [drv] + [os.path.join(csrc, s) for s in sources]:
            key = (f, tuple(defines))
            if key in objects:
                continue
            tag = os.path.splitext(os.path.basename(f))[0] + "".join(d.replace("-D", "_") for d in defines)
            jobs[key] = os.path.join(out_dir if f == drv else os.path.dirname(src), tag + ".o")

    def compile_one(item):
        (f, defines), obj = item
        subprocess.run([CXX, *flags, *defines, *inc, "-c", f, "-o", obj], check=True)

    if jobs:
        with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
            list(ex.map(compile_one, jobs.items()))
    for key, obj in jobs.items():
        if key[0] != drv:
            objects[key] = obj
    jobs.update({k: v for k, v in objects.items()})
    out = {}
    for name, (sources, defines) in variants.items():
        objs = [jobs[(os.path.join(ROOT, "tests", "wave_emu", driver), tuple(defines))]] + \
               [jobs[(os.path.join(csrc, s), tuple(defines))] for s in sources]
        exe = os.path.join(out_dir, f"{os.path.splitext(driver)[0]}_{name}")
        subprocess.run([CXX, "-pthread", *objs, "-o", exe], check=True)
        out[name] = exe
    return out
