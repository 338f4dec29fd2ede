"""A writer of seeded key part files restated from the format's specification (the reference's
hpc_gpu_port/seeded_keys.hpp:44-51): the tests build files with it independently of the engine's writer.

  char[8] "FSSMSKY1"; u32 version = 1; u32 expander = 1; u32 N; u32 sizeQ; u32 sizeP; u32 numPartQ;
  u32 numPerPartQ; u32 count; u32 keyTagLen; keyTag bytes; u64 moduli[sizeQ + sizeP];
  per key: u32 automorphism index; u8 seed[32]; u64 b[numPartQ][sizeQ + sizeP][N]   (all little-endian)
"""
import struct

import numpy as np

TAG_SKEY = 0x59454B53  # "SKEY" read little-endian: the third nonce word of the a-half expander


def part_bytes(N, moduli, size_q, size_p, num_part_q, num_per_part_q, key_tag, records, magic=b"FSSMSKY1",
               version=1, expander=1, count=None):
    """records: [(index, seed32, b as uint64 [num_part_q][size_q + size_p][N])]"""
    out = bytearray(magic)
    out += struct.pack("<9I", version, expander, N, size_q, size_p, num_part_q, num_per_part_q,
                       len(records) if count is None else count, len(key_tag))
    out += key_tag.encode()
    out += struct.pack(f"<{len(moduli)}Q", *moduli)
    for index, seed, b in records:
        out += struct.pack("<I", index)
        out += bytes(seed)
        out += np.ascontiguousarray(b, dtype="<u8").tobytes()
    return bytes(out)
