"""TEST INFRASTRUCTURE ONLY: rewrites copies of the library's HIP sources for
the CPU emulator (tests/wave_emu/hip/hip_runtime.h), leaving the originals
untouched:
  * `kernel<<<config>>>(args);`      -> `emu::launch_with([&] { kernel(args); }, config);`
  * `extern __shared__ T name[];`    -> `T* name = (T*)emu::dynamic_lds();`
  * `__shared__ T name[...];`        -> `static T name[...];` (one workgroup runs at a time)
usage: prep.py <repo root> <out dir>   (writes <out>/a/csrc/* and <out>/include/*)"""
import os
import re
import shutil
import sys

LAUNCH = re.compile(r"([A-Za-z_][\w:]*(?:<[^;{}]*?>)?)\s*<<<(.*?)>>>\s*\((.*?)\);", re.S)
ATTR = r"(?:__attribute__\(\((?:[^()]|\([^()]*\))*\)\)\s*)?"
EXTERN_SHARED = re.compile(r"extern\s+__shared__\s+" + ATTR + r"([\w: ]+?)\s+(\w+)\[\];")
SHARED = re.compile(r"__shared__\s+" + ATTR)


def rewrite(text: str) -> str:
    text = LAUNCH.sub(lambda m: f"emu::launch_with([&] {{ {m.group(1)}({m.group(3)}); }}, {m.group(2)});", text)
    text = EXTERN_SHARED.sub(lambda m: f"{m.group(1)}* {m.group(2)} = ({m.group(1)}*)emu::dynamic_lds();", text)
    text = SHARED.sub("static ", text)
    return text


def main(root: str, out: str) -> None:
    src = os.path.join(root, "tau.rs_amd", "csrc")
    dst = os.path.join(out, "a", "csrc")
    os.makedirs(dst, exist_ok=True)
    os.makedirs(os.path.join(out, "include"), exist_ok=True)
    shutil.copy(os.path.join(root, "include", "tau_moe.h"), os.path.join(out, "include", "tau_moe.h"))
    for name in os.listdir(src):
        if name.endswith((".hip", ".hpp")):
            text = open(os.path.join(src, name)).read()
            out_name = name[:-4] + ".cpp" if name.endswith(".hip") else name
            open(os.path.join(dst, out_name), "w").write(rewrite(text))


if __name__ == "__main__":
    main(sys.argv[1], sys.argv[2])
