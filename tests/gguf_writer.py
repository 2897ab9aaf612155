"""A minimal GGUF v3 writer for tests (written from the format description:
magic "GGUF", u32 version, u64 n_tensors, u64 n_kv, KVs, tensor infos, data
aligned to general.alignment).  Test infrastructure only."""
import struct

import numpy as np

# KV value types (gguf_type)
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f",
        BOOL: "<?", U64: "<Q", I64: "<q", F64: "<d"}


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(t, v):
    if t == STRING:
        return _str(v)
    if t == ARRAY:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        return out + b"".join(_value(et, x) for x in items)
    return struct.pack(_FMT[t], v)


def write_gguf(path, kvs, tensors, alignment=32, version=3):
    """kvs: [(key, type, value)]; tensors: [(name, dims (ne0 first), ggml type,
    bytes)].  Data offsets are aligned; general.alignment is written when
    `alignment` is not 32."""
    kvs = list(kvs)
    if alignment != 32:
        kvs.append(("general.alignment", U32, alignment))
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kvs))
    for key, t, v in kvs:
        head += _str(key) + struct.pack("<I", t) + _value(t, v)
    offs, off = [], 0
    for _, _, _, data in tensors:
        off = (off + alignment - 1) // alignment * alignment
        offs.append(off)
        off += len(data)
    for (name, dims, ttype, _), o in zip(tensors, offs):
        head += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", ttype, o)
    pad = (-len(head)) % alignment
    with open(path, "wb") as f:
        f.write(head + b"\0" * pad)
        pos = 0
        for (_, _, _, data), o in zip(tensors, offs):
            f.write(b"\0" * (o - pos))
            f.write(bytes(data))
            pos = o + len(data)


def expert_file(path, rng, n_layers, n_expert, hidden, n_ff, q6_down=(), alignment=32, extra_kvs=()):
    """Random Q4_K expert tensors blk.L.ffn_{gate,up,down}_exps; layers in
    q6_down get a Q6_K down projection.  Returns {(L, m): bytes [E][rows][...]}."""
    from sager_amd.synth import q4k_random_np, q6k_random_np
    kvs = [("general.architecture", STRING, "sage"), ("sage.block_count", U32, n_layers),
           ("sage.expert_count", U32, n_expert)] + list(extra_kvs)
    tensors, data = [], {}
    for L in range(n_layers):
        g = q4k_random_np(rng, n_expert * n_ff * hidden // 256)
        u = q4k_random_np(rng, n_expert * n_ff * hidden // 256)
        if L in q6_down:
            d, dt = q6k_random_np(rng, n_expert * hidden * n_ff // 256), 14
        else:
            d, dt = q4k_random_np(rng, n_expert * hidden * n_ff // 256), 12
        tensors += [(f"blk.{L}.ffn_gate_exps", (hidden, n_ff, n_expert), 12, g.tobytes()),
                    (f"blk.{L}.ffn_up_exps", (hidden, n_ff, n_expert), 12, u.tobytes()),
                    (f"blk.{L}.ffn_down_exps", (n_ff, hidden, n_expert), dt, d.tobytes())]
        data[(L, 0)], data[(L, 1)], data[(L, 2)] = g, u, d
    tensors.append(("token_embd.weight", (hidden, 4), 0, np.zeros(4 * hidden, np.float32).tobytes()))
    write_gguf(path, kvs, tensors, alignment=alignment)
    return data
