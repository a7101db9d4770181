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


# Inline assembly of grouped_gemm.hip's direct-to-LDS copies, replaced by the
# emulator's copy (same operands: the per-lane source and the LDS destination
# whose first lane's address is the wave's base) and its barrier.
ASM = [
    (re.compile(r'asm volatile\("s_waitcnt vmcnt\(%0\)"[^;]*;'), ""),
    (re.compile(r'asm volatile\("s_mov_b32 m0, %1\\n\\ts_nop 0\\n\\tglobal_load_lds_dwordx4 %0, off"[^;]*;'),
     "emu::dma16(src, lds); (void)base;"),
    (re.compile(r'asm volatile\("s_mov_b32 m0, %2\\n\\ts_nop 0\\n\\tglobal_load_lds_dwordx4 %0, %1"[^;]*;'),
     "emu::dma16((const uint16_t*)((const char*)(uintptr_t)gs + off_bytes), lds); (void)lbase;"),
    (re.compile(r'asm volatile\("s_waitcnt lgkmcnt\(0\)\\n\\ts_barrier"[^;]*;'), "__syncthreads();"),
]


def rewrite(text: str) -> str:
    for pattern, repl in ASM:
        text = pattern.sub(repl, text)
    if "asm volatile" in text:
        raise RuntimeError("unhandled inline assembly")
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
