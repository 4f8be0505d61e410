"""numpy statement of the packed weight layout of ihip_pack_weights (test
infrastructure): chunk (tile t, unit u) at (t * n_units + u) * 16 * UB, lane
l = n + 16 g of row n. Used to pin the device packer byte for byte. Q4_K swaps
bytes 1 and 2 of each quant dword; Q6_K regroups each lane's quant bits into
6-bit fields (q6_words); the other bytes are moved whole."""
import numpy as np

from inferno_hip import formats as F


def unit_bytes(qt):
    return 8 * 34 if qt == F.Q8_0 else F.BLOCK_BYTES[qt]


def q6_words(a, b, h):
    """The three Q6_K words of one lane and group from its GGUF bytes (ql
    a[j] = ql[p + j], b[j] = ql[p + 32 + j], qh h[j]), element by element:
    value j of the group's sub-block qq is nibble qq >> 1 of a[j] (qq even)
    or b[j] with bits 2 qq, 2 qq + 1 of h[j] above it; pair (qq, t) is
    values 2t, 2t + 1, placed at bits o and 16 + o of a word."""
    v = [[((int(a[j]) if qq % 2 == 0 else int(b[j])) >> (4 * (qq >> 1)) & 0xF) | ((int(h[j]) >> (2 * qq) & 3) << 4)
          for j in range(4)] for qq in range(4)]

    def put(qq, t, o):
        return (v[qq][2 * t] << o) | (v[qq][2 * t + 1] << (16 + o))

    A = put(0, 0, 0) | put(0, 1, 6) | ((v[3][0] & 0xF) << 12) | ((v[3][1] & 0xF) << 28)
    B = put(1, 0, 0) | put(1, 1, 6) | ((v[3][2] & 0xF) << 12) | ((v[3][3] & 0xF) << 28)
    C = (put(2, 0, 0) | ((v[3][0] >> 4) << 6) | ((v[3][1] >> 4) << 22) | ((v[3][2] >> 4) << 8) |
         ((v[3][3] >> 4) << 24) | put(2, 1, 10))
    return A, B, C


def pack_ref(qt, w, N, K):
    bb = F.BLOCK_BYTES[qt]
    row_bytes = K // F.BLOCK_ELEMS[qt] * bb
    n_units = (K + 255) // 256
    n_tiles = (N + 15) // 16
    UB = unit_bytes(qt)
    CH = 16 * UB
    rows = np.zeros((n_tiles * 16, n_units * UB), np.uint8)  # zero-padded rows / units
    rows[:N, :row_bytes] = np.asarray(w, np.uint8).reshape(N, row_bytes)
    out = np.zeros((n_tiles, n_units, CH), np.uint8)
    for t in range(n_tiles):
        for u in range(n_units):
            ch = out[t, u]
            for l in range(64):
                n, g = l & 15, l >> 4
                src = rows[16 * t + n, u * UB:(u + 1) * UB]
                if qt == F.Q4_K:
                    for i in range(2):  # bytes 1 and 2 of each quant dword swapped
                        q = src[16 + 64 * i + 16 * g:32 + 64 * i + 16 * g].reshape(4, 4)[:, [0, 2, 1, 3]]
                        ch[1024 * i + 16 * l:1024 * i + 16 * l + 16] = q.reshape(16)
                    if g == 0:
                        ch[2048 + 16 * n:2064 + 16 * n] = src[:16]
                elif qt == F.Q5_K:
                    for i in range(2):
                        ch[1024 * i + 16 * l:1024 * i + 16 * l + 16] = src[48 + 64 * i + 16 * g:64 + 64 * i + 16 * g]
                    if g < 2:
                        o = 2048 + 16 * (n + 16 * g)
                        ch[o:o + 16] = src[16 + 16 * g:32 + 16 * g]
                    if g == 0:
                        ch[2560 + 16 * n:2576 + 16 * n] = src[:16]
                elif qt == F.Q6_K:
                    for i in range(4):
                        p = 64 * (i >> 1) + 16 * (i & 1) + 4 * g
                        q = 128 + 32 * (i >> 1) + 16 * (i & 1) + 4 * g
                        words = q6_words(src[p:p + 4], src[p + 32:p + 36], src[q:q + 4])
                        for k in range(3):
                            ch[1024 * k + 16 * l + 4 * i:1024 * k + 16 * l + 4 * i + 4] = \
                                np.frombuffer(int(words[k]).to_bytes(4, "little"), np.uint8)
                    if g == 0:
                        ch[3072 + 16 * n:3088 + 16 * n] = src[192:208]
                        ch[3328 + 2 * n:3330 + 2 * n] = src[208:210]
                else:
                    for i in range(4):
                        for j in range(2):
                            for h in range(2):
                                b = 2 * i + j
                                o = 1024 * i + 16 * l + 8 * j + 4 * h
                                s = 34 * b + 2 + 4 * (g + 4 * h)
                                ch[o:o + 4] = src[s:s + 4]
                    if g == 0:
                        for b in range(8):
                            ch[4096 + 16 * n + 2 * b:4098 + 16 * n + 2 * b] = src[34 * b:34 * b + 2]
    return out.reshape(-1)
