"""Build guard for the persistent decode kernel's code shape.

The kernel (decode_fused.hip) depends on properties the compiler could
silently take away:
  * no scratch memory and no dynamic stack: a call frame or a spilled vector
    register would put private-memory traffic on every step's critical path;
  * no calls: every helper (the polls included) is inlined, so the weight
    registers held across them need no call-preserved registers and the
    compiler's waits for weight rows held in registers stay exact;
  * the kernarg-segment intrinsic is read once, in the kernel's own body: the
    compiler lowers it to a null pointer in any function that is not a
    kernel, so a helper that called it and got outlined would read launch
    arguments from address 0;
  * every global store of more than 64 data bits written as inline assembly
    is followed at once by s_nop 1 or longer: such a store reads its data
    registers after issue, a VALU write to them needs two wait states on
    this chip, and the compiler cannot insert them for a store it does not
    see (without them the store can write the registers' next values);
  * every matrix-core instruction runs with the whole wave enabled: its
    operands come from all 64 lanes, so one placed inside a lane-divergent
    branch (after an s_and_saveexec before the branch's exec restore)
    would combine operands that only some lanes loaded.

The script compiles decode_fused.hip for the device with the compiler's
resource-usage remarks, writes the device assembly next to the objects, and
exits non-zero (naming the property) when any decode_flow_kernel instance
breaks one of them. The Makefile runs it before linking the library.

Usage: python3 check_code_shape.py HIPCC OUT_DIR -- <hipcc flags>
"""
import re
import subprocess
import sys

SRC = "decode_fused.hip"
KERNEL = "decode_flow_kernel"
ALLOWED_CALLEES = ()


def fail(msg):
    print(f"check_code_shape: {msg}", file=sys.stderr)
    sys.exit(1)


def check_source():
    text = open(SRC).read()
    uses = [m.start() for m in re.finditer(r"__builtin_amdgcn_kernarg_segment_ptr\s*\(", text)]
    if len(uses) != 1:
        fail(f"{SRC} reads the kernarg-segment pointer {len(uses)} times; it must be read once, in the "
             f"kernel body")
    body = text.find(f"void {KERNEL}(")
    end = text.find("\n}\n", body)
    if body < 0 or not body < uses[0] < end:
        fail(f"{SRC}: the kernarg-segment pointer is read outside {KERNEL}'s body")


def remarks(stderr):
    """{function name: {key: value}} from -Rpass-analysis=kernel-resource-usage."""
    out, cur = {}, None
    for line in stderr.splitlines():
        m = re.search(r"remark:\s+Function Name: (\S+)", line)
        if m:
            cur = out.setdefault(m.group(1), {})
            continue
        m = re.search(r"remark:\s+([A-Za-z][A-Za-z \[\]/]*?): (\S+) \[-Rpass-analysis", line)
        if m and cur is not None:
            cur[m.group(1).strip()] = m.group(2)
    return out


def functions(asm):
    """{symbol: body lines} for every function in the device assembly."""
    names = set(re.findall(r"^\s*\.type\s+([\w.$]+),@function", asm, re.M))
    out, cur = {}, None
    for line in asm.splitlines():
        lab = re.match(r"^([\w.$]+):", line)
        if lab and lab.group(1) in names:
            cur = out.setdefault(lab.group(1), [])
            continue
        if line.startswith(".Lfunc_end"):
            cur = None
            continue
        if cur is not None:
            cur.append(line)
    return out, names


def main():
    if len(sys.argv) < 4 or sys.argv[3] != "--":
        fail("usage: check_code_shape.py HIPCC OUT_DIR -- <flags>")
    hipcc, out_dir, flags = sys.argv[1], sys.argv[2], sys.argv[4:]
    check_source()
    asm_path = f"{out_dir}/decode_fused.device.s"
    cmd = [hipcc, *flags, "--cuda-device-only", "-S", "-Rpass-analysis=kernel-resource-usage", SRC, "-o", asm_path]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stderr)
        fail("device compile failed")
    res = {k: v for k, v in remarks(r.stderr).items() if KERNEL in k}
    if not res:
        fail(f"no resource-usage remarks for {KERNEL}")
    for name, kv in res.items():
        if kv.get("ScratchSize [bytes/lane]") != "0":
            fail(f"{name}: scratch size {kv.get('ScratchSize [bytes/lane]')} bytes/lane (must be 0)")
        if kv.get("Dynamic Stack") != "False":
            fail(f"{name}: dynamic stack")
        if kv.get("VGPRs Spill") != "0":
            fail(f"{name}: {kv.get('VGPRs Spill')} vector registers spilled")
    funcs, names = functions(open(asm_path).read())
    kernels = [f for f in funcs if KERNEL in f]
    if len(kernels) != len(res):
        fail(f"{len(kernels)} {KERNEL} bodies in the assembly, {len(res)} in the remarks")
    for k in kernels:
        callees = set()
        for line in funcs[k]:
            for sym in re.findall(r"([\w.$]+)@(?:rel32|gotpcrel32)@lo", line):
                if sym in names or "@gotpcrel" in line:
                    callees.add(sym)
        bad = [c for c in callees if not (ALLOWED_CALLEES and c.startswith(ALLOWED_CALLEES))]
        if bad or any("s_swappc" in line for line in funcs[k]):
            fail(f"{k} calls {bad or 'a function'}: every helper must be inlined")
        wide = check_wide_stores(funcs[k])
        if wide:
            fail(f"{k}: a store of more than 64 data bits is not followed by s_nop 1: {wide}")
        masked = check_mfma_exec(funcs[k])
        if masked:
            fail(f"{k}: a matrix-core instruction inside a lane-divergent branch: {masked}")
    print(f"check_code_shape: {len(kernels)} {KERNEL} instances: no scratch, no dynamic stack, no vector "
          f"spills, no calls, wide stores padded, matrix-core products on whole waves")


def check_mfma_exec(body):
    """The first v_mfma whose closest preceding exec change in the code
    layout narrows exec (s_and_saveexec) rather than restoring it, or None."""
    last = ""
    for ln in body:
        ins = ln.split(";")[0].strip()
        if re.match(r"s_and_saveexec_b64|s_or_b64 exec, exec|s_andn2_b64 exec|s_mov_b64 exec|s_xor_b64 exec|"
                    r"s_and_b64 exec", ins):
            last = ins
        elif ins.startswith("v_mfma") and last.startswith("s_and_saveexec"):
            return ins
    return None


def check_wide_stores(body):
    """The first wide store (dwordx3/x4) whose next instruction is not an
    s_nop of at least 2 wait states, or None."""
    insts = [ln.split(";")[0].strip() for ln in body]
    insts = [i for i in insts if i and not i.startswith(".") and not i.endswith(":")]
    for n, ins in enumerate(insts):
        if re.match(r"(global|buffer|flat)_store_dwordx[34]\b", ins):
            nxt = insts[n + 1] if n + 1 < len(insts) else ""
            m = re.match(r"s_nop\s+(\d+)", nxt)
            if not m or int(m.group(1)) < 1:
                return ins
    return None


if __name__ == "__main__":
    main()
