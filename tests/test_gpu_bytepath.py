"""Device byte path against the oracle (MI355X): XXH64 digest kernel, checkpoint-parallel verify, unit scatter, synth.

Every comparison is bit-exact (integer / byte work). Inputs are seeded; the oracle runs on the same bytes on the CPU.
"""
import ctypes as C

import numpy as np
import pytest
import xxhash

import oracle
from oracle import synth

pytestmark = pytest.mark.gpu


def _pack(gpu, arrays, align=256):
    """Upload arrays into one device buffer at `align`-aligned offsets; returns (buffer, [(ptr, bytes)])."""
    offs, pos = [], 0
    for a in arrays:
        offs.append(pos)
        pos += (a.nbytes + align - 1) // align * align
    buf = gpu.DeviceBuffer(max(pos, align))
    for a, o in zip(arrays, offs):
        if a.nbytes:
            buf.upload(a, o)
    return buf, [(buf.ptr + o, a.nbytes) for a, o in zip(arrays, offs)]


def test_digest_every_small_length(gpu, oracle):
    rng = np.random.default_rng(1)
    arrays = [rng.integers(0, 256, n, dtype=np.uint8) for n in range(0, 300)]
    buf, ext = _pack(gpu, arrays)
    units = [gpu.make_unit([e]) for e in ext]
    got = gpu.device_digests(units)
    want = [oracle.xxh64(a) for a in arrays]
    assert got == want
    assert want[3] == xxhash.xxh64_intdigest(arrays[3].tobytes())


def test_digest_multi_extent_units(gpu, oracle):
    rng = np.random.default_rng(2)
    shapes = [[1 << 20] * 3, [4096, 32, 7], [96, 64, 32, 33], [32 * 1000, 1], [1 << 16]]
    all_arrays, groups = [], []
    for sh in shapes:
        g = [rng.integers(0, 256, s, dtype=np.uint8) for s in sh]
        groups.append(g)
        all_arrays += g
    buf, ext = _pack(gpu, all_arrays)
    units, k = [], 0
    for g in groups:
        units.append(gpu.make_unit(ext[k:k + len(g)]))
        k += len(g)
    got = gpu.device_digests(units)
    assert got == [oracle.xxh64_extents(g) for g in groups]


def test_digest_many_units_batch(gpu, oracle):
    # 2048 units of 4 KiB + ragged tails: the batched (HBM-bound) regime
    rng = np.random.default_rng(3)
    arrays = [rng.integers(0, 256, 4096 + (i % 37), dtype=np.uint8) for i in range(2048)]
    buf, ext = _pack(gpu, arrays)
    got = gpu.device_digests([gpu.make_unit([e]) for e in ext])
    assert got == [oracle.xxh64(a) for a in arrays]


def _verify(gpu, ext_groups, states_list, digests, seg):
    units, first = [], 0
    state_bufs = []
    for ext, st, dg in zip(ext_groups, states_list, digests):
        sb = gpu.DeviceBuffer(max(st.nbytes, 8))
        sb.upload(st)
        state_bufs.append(sb)
        vu = gpu.TsaVerifyUnit()
        for i, (p, b) in enumerate(ext):
            vu.ext[i].ptr = p
            vu.ext[i].bytes = b
        vu.n_ext = len(ext)
        vu.seg_first = first
        vu.states = sb.ptr
        vu.digest = dg
        vu.total = sum(b for _, b in ext)
        first += len(st) // 4
        units.append(vu)
    table = gpu.upload_struct_array(units)
    fail = gpu.DeviceBuffer(4 * len(units))
    fail.upload(np.zeros(len(units), dtype=np.uint32))
    gpu.check(gpu.lib().tsa_xxh64_verify(C.c_void_p(table.ptr), len(units), first, seg, C.c_void_p(fail.ptr), None))
    gpu.check(gpu.lib().tsa_stream_sync(None))
    return fail.download(4 * len(units)).view(np.uint32)


@pytest.mark.parametrize("seg,align", [(1024, 256), (1536, 256), (8192, 256), (65536, 256),
                                       # 2 KiB segments: waves of whole 16-byte aligned segments stream through LDS,
                                       # the rest (the 31-byte and empty units, 8-byte aligned extents) run the chain
                                       (2048, 256), (2048, 8)])
def test_verify_checkpoint_parallel(gpu, oracle, seg, align):
    rng = np.random.default_rng(seg)
    shapes = [[1 << 20] * 3, [(1 << 18) + 32 * 5, 4096, 1000], [31], [0], [32 * 3 + 5], [1 << 16, 1 << 16]]
    groups = [[rng.integers(0, 256, s, dtype=np.uint8) for s in sh] for sh in shapes]
    flat = [a for g in groups for a in g]
    buf, ext = _pack(gpu, flat, align)
    ext_groups, k = [], 0
    for g in groups:
        ext_groups.append(ext[k:k + len(g)])
        k += len(g)
    states, digests = [], []
    for g in groups:
        st, dg = oracle.checkpoints(g, seg)
        # the product's host checkpoints equal the oracle's, bit for bit
        st2, dg2 = gpu.host_checkpoints(g, seg)
        assert np.array_equal(st, st2) and dg == dg2 == xxhash.xxh64_intdigest(b"".join(a.tobytes() for a in g))
        states.append(st)
        digests.append(dg)
    assert list(_verify(gpu, ext_groups, states, digests, seg)) == [0] * len(groups)
    # one flipped byte inside unit 1's second extent (and one in unit 0's last tail byte): only those units fail
    p, b = ext_groups[1][1]
    one = np.frombuffer(np.array([255 - groups[1][1][17]], dtype=np.uint8).tobytes(), dtype=np.uint8)
    gpu.check(gpu.lib().tsa_memcpy(C.c_void_p(p + 17), one.ctypes.data_as(C.c_void_p), 1, 0, None))
    p0, b0 = ext_groups[0][2]
    one0 = np.array([255 - groups[0][2][b0 - 1]], dtype=np.uint8)
    gpu.check(gpu.lib().tsa_memcpy(C.c_void_p(p0 + b0 - 1), one0.ctypes.data_as(C.c_void_p), 1, 0, None))
    gpu.check(gpu.lib().tsa_stream_sync(None))
    res = _verify(gpu, ext_groups, states, digests, seg)
    assert [int(x != 0) for x in res] == [1, 1, 0, 0, 0, 0]


@pytest.mark.parametrize("parts,seg", [([64 * 1024] * 3, 2048), ([2048, 4096 + 32, 1000], 1024), ([96], 1024),
                                       ([8454144, 64 * 1024, 4 * 1024 * 1024], 2048)])
def test_scatter_verify_slots_arena(gpu, oracle, parts, seg):
    """tsa_xxh64_scatter_verify_slots (the staged units' scatter fused with their check): units back to back in HBM
    staging go to their arena slots byte for byte (a last part's tail under 32 bytes included) and pass; a flipped
    staged byte - a part's first, the unit's last (in the tail) - fails only its unit, whose slot then holds the
    flipped bytes as staged."""
    rng = np.random.default_rng(len(parts) * seg + parts[0] + 7)
    ub = sum(parts)
    slots_n, keys_n = 6, 5
    arena = [gpu.DeviceBuffer(slots_n * pb) for pb in parts]
    data = {k: [rng.integers(0, 256, pb, dtype=np.uint8) for pb in parts] for k in range(keys_n)}
    placed = {0: 3, 2: 0, 4: 5, 1: 1}  # key -> slot, in the order the units are staged
    n_ck = len(oracle.checkpoints(data[0], seg)[0]) // 4
    states = np.zeros((keys_n, n_ck, 4), dtype=np.uint64)
    digests = np.zeros(keys_n, dtype=np.uint64)
    for k in range(keys_n):
        st, dg = oracle.checkpoints(data[k], seg)
        states[k] = st.reshape(n_ck, 4)
        digests[k] = dg
    st_dev = gpu.DeviceBuffer(states.nbytes)
    st_dev.upload(states)
    dg_dev = gpu.DeviceBuffer(digests.nbytes)
    dg_dev.upload(digests)
    staged = np.concatenate([np.concatenate(data[k]) for k in placed])
    src = gpu.DeviceBuffer(staged.nbytes)
    a = gpu.TsaArenaVerify()
    for p, (buf, pb) in enumerate(zip(arena, parts)):
        a.arena[p] = buf.ptr
        a.part_bytes[p] = pb
    a.n_parts, a.seg_bytes, a.states_dev, a.digests_dev = len(parts), seg, st_dev.ptr, dg_dev.ptr
    keys = (C.c_uint32 * len(placed))(*placed.keys())
    slots = (C.c_int32 * len(placed))(*placed.values())
    fail = gpu.DeviceBuffer(4 * len(placed))

    def run(bytes_):
        src.upload(bytes_)
        fail.upload(np.zeros(len(placed), dtype=np.uint32))
        gpu.check(gpu.lib().tsa_xxh64_scatter_verify_slots(C.byref(a), keys, slots, len(placed), C.c_void_p(src.ptr),
                                                           C.c_void_p(fail.ptr), None))
        gpu.check(gpu.lib().tsa_stream_sync(None))
        return list(fail.download(4 * len(placed)).view(np.uint32))

    def slot_bytes(sl):
        return np.concatenate([buf.download(pb, sl * pb) for buf, pb in zip(arena, parts)])

    assert run(staged) == [0] * len(placed)
    for i, (k, sl) in enumerate(placed.items()):
        assert np.array_equal(slot_bytes(sl), staged[i * ub:(i + 1) * ub]), (k, sl)
    bad = staged.copy()
    bad[2 * ub - 1] ^= 0xFF           # unit 1 (key 2): its last byte
    bad[3 * ub + (parts[0] if len(parts) > 1 else 1)] ^= 0x01  # unit 3 (key 1): its second part's first byte
    got = run(bad)
    assert got[0] == 0 and got[1] != 0 and got[2] == 0 and got[3] != 0, got
    assert np.array_equal(slot_bytes(placed[2]), bad[ub:2 * ub])  # (written as staged, and flagged)


@pytest.mark.parametrize("parts,seg", [([64 * 1024] * 3, 8192), ([2048, 4096 + 32, 1000], 1024), ([96], 1024),
                                       # 2 KiB segments and 16-byte aligned parts: the LDS-streamed kernel (whole
                                       # segments; short last segments and a 16-byte tail; one- and two-stripe
                                       # segments; many workgroups with a partly dead last wave)
                                       ([64 * 1024] * 3, 2048), ([2048, 4096 + 32, 1008], 2048), ([96], 2048),
                                       ([64, 80], 2048), ([8454144, 64 * 1024 + 32, 4 * 1024 * 1024 + 16], 2048),
                                       # 2 KiB segments, a last part of 1000 bytes: slots 1 and 5 are not 16-byte
                                       # aligned, so the launch takes the chain kernel
                                       ([2048, 4096 + 32, 1000], 2048)])
def test_verify_slots_arena(gpu, oracle, parts, seg):
    """tsa_xxh64_verify_slots (the device-gated check): keys in arena slots, by value; against the oracle's
    checkpoints and XXH64; then one flipped byte fails only its unit."""
    rng = np.random.default_rng(len(parts) * seg + parts[0])
    slots_n, keys_n = 6, 5
    arena = [gpu.DeviceBuffer(slots_n * pb) for pb in parts]
    data = {k: [rng.integers(0, 256, pb, dtype=np.uint8) for pb in parts] for k in range(keys_n)}
    placed = {0: 3, 2: 0, 4: 5, 1: 1}  # key -> slot
    for k, sl in placed.items():
        for p, (buf, pb) in enumerate(zip(arena, parts)):
            buf.upload(data[k][p], sl * pb)
    n_ck = len(oracle.checkpoints(data[0], seg)[0]) // 4
    states = np.zeros((keys_n, n_ck, 4), dtype=np.uint64)
    digests = np.zeros(keys_n, dtype=np.uint64)
    for k in range(keys_n):
        st, dg = oracle.checkpoints(data[k], seg)
        states[k] = st.reshape(n_ck, 4)
        digests[k] = dg
        assert dg == xxhash.xxh64_intdigest(b"".join(a.tobytes() for a in data[k]))
    st_dev = gpu.DeviceBuffer(states.nbytes)
    st_dev.upload(states)
    dg_dev = gpu.DeviceBuffer(digests.nbytes)
    dg_dev.upload(digests)
    a = gpu.TsaArenaVerify()
    for p, (buf, pb) in enumerate(zip(arena, parts)):
        a.arena[p] = buf.ptr
        a.part_bytes[p] = pb
    a.n_parts, a.seg_bytes, a.states_dev, a.digests_dev = len(parts), seg, st_dev.ptr, dg_dev.ptr
    keys = (C.c_uint32 * len(placed))(*placed.keys())
    slots = (C.c_int32 * len(placed))(*placed.values())
    fail = gpu.DeviceBuffer(4 * len(placed))

    def run():
        fail.upload(np.zeros(len(placed), dtype=np.uint32))
        gpu.check(gpu.lib().tsa_xxh64_verify_slots(C.byref(a), keys, slots, len(placed), C.c_void_p(fail.ptr), None))
        gpu.check(gpu.lib().tsa_stream_sync(None))
        return list(fail.download(4 * len(placed)).view(np.uint32))

    assert run() == [0] * len(placed)
    # key 4 (slot 5): flip a byte of its last part's last byte; key 2 (slot 0): its first part's first byte
    last = len(parts) - 1
    one = np.array([255 - data[4][last][-1]], dtype=np.uint8)
    arena[last].upload(one, 5 * parts[last] + parts[last] - 1)
    assert run() == [0, 0, 1, 0]
    arena[0].upload(np.array([255 - data[2][0][0]], dtype=np.uint8), 0)
    assert run() == [0, 1, 1, 0]


def test_scatter_parts(gpu):
    rng = np.random.default_rng(9)
    part_bytes = [(1 << 20) + 256, 4096, 3 * 16384 + 16]
    units = [rng.integers(0, 256, sum(part_bytes), dtype=np.uint8) for _ in range(3)]
    src_buf, src_ext = _pack(gpu, units)
    dst = gpu.DeviceBuffer(3 * sum(((b + 255) // 256) * 256 for b in part_bytes) + 4096)
    jobs, first, dst_ptrs = [], 0, []
    pos = 0
    for (sp, _), u in zip(src_ext, units):
        j = gpu.TsaScatterJob()
        j.src = sp
        ptrs = []
        for i, b in enumerate(part_bytes):
            j.dst[i] = dst.ptr + pos
            j.bytes[i] = b
            ptrs.append(pos)
            pos += (b + 255) // 256 * 256
        j.n_parts = len(part_bytes)
        j.block_first = first
        first += gpu.lib().tsa_scatter_blocks((C.c_uint64 * 3)(*part_bytes), 3)
        jobs.append(j)
        dst_ptrs.append(ptrs)
    table = gpu.upload_struct_array(jobs)
    gpu.check(gpu.lib().tsa_scatter(C.c_void_p(table.ptr), len(jobs), first, None))
    gpu.check(gpu.lib().tsa_stream_sync(None))
    host = dst.download()
    for u, ptrs in zip(units, dst_ptrs):
        off = 0
        for b, p in zip(part_bytes, ptrs):
            assert np.array_equal(host[p:p + b], u[off:off + b])
            off += b


def test_synth_uniform_matches_oracle(gpu):
    n = 1 << 20
    buf = gpu.DeviceBuffer(n)
    gpu.check(gpu.lib().tsa_synth(C.c_void_p(buf.ptr), n, 1234, 77, 4096, 0, C.c_float(0.0), None))
    gpu.check(gpu.lib().tsa_stream_sync(None))
    assert np.array_equal(buf.download(), synth.uniform_bytes(1234, 77, 4096, n))


def test_synth_q4_blocks_match_oracle(gpu):
    """Q4 blocks are integer arithmetic: bit-exact, including a start inside a block (offset 4096 = block 227 + 10)."""
    n = (1 << 20) + 8
    buf = gpu.DeviceBuffer(n)
    gpu.check(gpu.lib().tsa_synth(C.c_void_p(buf.ptr), n, 99, 5, 4096, 2, C.c_float(0.0), None))
    gpu.check(gpu.lib().tsa_stream_sync(None))
    assert np.array_equal(buf.download(), synth.q4_blocks(99, 5, 4096, n))


def test_synth_bf16_normal(gpu):
    n = 1 << 22
    buf = gpu.DeviceBuffer(n)
    gpu.check(gpu.lib().tsa_synth(C.c_void_p(buf.ptr), n, 5, 1, 0, 1, C.c_float(0.02), None))
    gpu.check(gpu.lib().tsa_stream_sync(None))
    got = buf.download().view(np.uint16)
    want = synth.bf16_normal(5, 1, 0, n, 0.02).view(np.uint16)
    # the same Box-Muller in float32: equal except for rare last-ulp rounding differences of log/sin/cos
    assert np.mean(got == want) > 0.999
    x = (got.astype(np.uint32) << 16).view(np.float32)
    assert abs(float(x.mean())) < 1e-3 and abs(float(x.std()) - 0.02) < 1e-3
