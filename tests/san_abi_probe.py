"""Host-side probe of the C-ABI for the sanitizer-built library (libwide_hip_san.so).

Run by tests/test_abi_sanitized.py in a child process that preloads the AddressSanitizer
runtime (the Python interpreter itself is not instrumented); not collected by pytest.  It needs
no GPU: every entry point declared in include/wc_abi.h is called with NULL, zero-filled,
0xFF-filled and random arguments (a fixed seed), so the argument checks, size arithmetic and
error reporting of the host code run under AddressSanitizer and UndefinedBehaviorSanitizer.
Device pointers are never dereferenced on the host; the only host arrays an entry point reads
(wc_pack_rows' source tables) are given buffers large enough for the counts passed with them;
stream arguments are always NULL (the HIP runtime dereferences a stream handle).

usage: python san_abi_probe.py <library> <wc_abi.h> <iterations> <package dir>
"""

import ctypes
import random
import re
import sys


def prototypes(header: str):
    text = re.sub(r"/\*.*?\*/", "", open(header).read(), flags=re.S)
    out = []
    for m in re.finditer(r"(int32_t|int64_t|const char\s*\*|void)\s+(wc_\w+)\s*\(([^;]*?)\)\s*;", text, flags=re.S):
        ret, name, params = m.group(1), m.group(2), " ".join(m.group(3).split())
        plist = [] if params.strip() in ("", "void") else [p.strip() for p in params.split(",")]
        out.append((ret, name, plist))
    return out


def ctype_of(param: str):
    if "*" in param:
        return ctypes.c_void_p
    if param.startswith("int64_t"):
        return ctypes.c_int64
    if param.startswith("int32_t"):
        return ctypes.c_int32
    if param.startswith("float"):
        return ctypes.c_float
    if param.startswith("double"):
        return ctypes.c_double
    raise ValueError(param)


def main() -> int:
    lib = ctypes.CDLL(sys.argv[1])
    protos = prototypes(sys.argv[2])
    iters = int(sys.argv[3])
    rng = random.Random(20261202)
    rets = {"int32_t": ctypes.c_int32, "int64_t": ctypes.c_int64, "void": None}
    fns = []
    for ret, name, plist in protos:
        f = getattr(lib, name)
        f.restype = ctypes.c_char_p if "char" in ret else rets[ret]
        f.argtypes = [ctype_of(p) for p in plist]
        fns.append((name, plist, f))
    assert len(fns) >= 25, [n for n, _, _ in fns]

    struct_bytes = 4096
    zero = ctypes.create_string_buffer(struct_bytes)
    ones = ctypes.create_string_buffer(b"\xff" * struct_bytes, struct_bytes)
    table = ctypes.create_string_buffer(1 << 16)             # host tables of up to 8192 entries
    ints = [0, 1, 2, 3, 7, 16, 64, 512, -1, -7, 1 << 20, (1 << 31) - 1, -(1 << 31), 1 << 40, -(1 << 62), (1 << 63) - 1]
    floats = [0.0, 1e-5, -1.0, float("nan"), float("inf")]

    def rand_struct():
        return ctypes.create_string_buffer(bytes(rng.getrandbits(8) for _ in range(struct_bytes)), struct_bytes)

    calls = 0
    for it in range(iters):
        for name, plist, f in fns:
            args = []
            host_table = name == "wc_pack_rows"
            for p in plist:
                pname = p.split()[-1].lstrip("*")
                t = ctype_of(p)
                if pname == "stream":
                    args.append(None)
                elif t is ctypes.c_void_p:
                    if "args" in p:                            # a struct read on the host
                        args.append(rng.choice([None, zero, ones, rand_struct()]))
                    elif host_table and pname in ("srcs", "src_row_stride_bytes"):
                        args.append(rng.choice([None, table]))
                    else:                                      # a device pointer: never dereferenced here
                        args.append(rng.choice([None, 16, 0x7F0000000000 + 256 * rng.randrange(1 << 20)]))
                elif t in (ctypes.c_float, ctypes.c_double):
                    args.append(rng.choice(floats))
                else:
                    v = rng.choice(ints) if rng.random() < 0.7 else rng.randrange(-100, 100000)
                    if host_table and pname == "n":
                        v = rng.choice([0, 1, 3, 64, 8192, -1])   # within the table buffer
                    if t is ctypes.c_int32:
                        v = max(min(v, (1 << 31) - 1), -(1 << 31))
                    args.append(v)
            f(*args)
            calls += 1
            msg = lib.wc_last_error()
            assert msg is None or isinstance(msg, bytes)
    calls += near_valid(lib, fns, rng, iters)
    print(f"san_abi_probe: {calls} calls over {len(fns)} entry points, no sanitizer report", flush=True)
    return 0


# the C structs an entry point reads, by the ctypes classes of the library's own binding
STRUCTS = {"wc_rnn_args": "_RnnArgs", "wc_gemm_args": "_GemmArgs", "wc_mlp2_args": "_Mlp2Args",
           "wc_conv_args": "_ConvArgs", "wc_conv3d_args": "_Conv3dArgs", "wc_attn_args": "_AttnArgs",
           "wc_self_attn_args": "_SelfAttnArgs"}


def near_valid(lib, fns, rng, iters: int) -> int:
    """Struct arguments with plausible sizes, valid dtype / cell / act codes and 4 KB-aligned
    (fake) device addresses, one field in five set to an extreme value: these pass the first
    checks and reach the planning code behind them (tile plans, grids, workspace layouts).
    Without a GPU every launch fails and reports an error."""
    sys.path.insert(0, sys.argv[4])
    from wide_compiler import _hip   # the ctypes struct classes (no library call is made here)

    plausible = [0, 1, 2, 3, 4, 7, 8, 16, 32, 33, 64, 128, 256, 384, 512, 768, 1024, 4096]
    extreme = [-1, -(1 << 31), (1 << 31) - 1, 1 << 32, 1 << 40, (1 << 63) - 1, -(1 << 63)]
    calls = 0
    for _ in range(iters):
        for name, plist, f in fns:
            st = next((k for k in STRUCTS if any(k in p for p in plist)), None)
            if st is None:
                continue
            a = getattr(_hip, STRUCTS[st])()
            for fname, ftype in a._fields_:
                if ftype is ctypes.c_void_p:
                    v = None if rng.random() < 0.1 else 0x7F0000000000 + 4096 * rng.randrange(1 << 16)
                elif ftype in (ctypes.c_float, ctypes.c_double):
                    v = rng.choice([1e-5, 0.125, 1.0])
                elif "dtype" in fname:
                    v = rng.choice([0, 1, 2, 0, 1, 2, 9])
                elif fname in ("cell", "act", "relu", "causal"):
                    v = rng.choice([0, 1, 0, 1, 3])
                else:
                    v = rng.choice(extreme) if rng.random() < 0.2 else rng.choice(plausible)
                    if ftype is ctypes.c_int32:
                        v = max(min(v, (1 << 31) - 1), -(1 << 31))
                setattr(a, fname, v)
            args = [ctypes.byref(a) if st in p else None for p in plist]
            f(*args)
            calls += 1
    return calls


if __name__ == "__main__":
    sys.exit(main())
