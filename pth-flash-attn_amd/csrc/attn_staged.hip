// attn_staged.hip -- the paged attention kernels with register-staged loads
// (block size a multiple of 16, cell view of the cache, D = 128): the
// long-row decode, verify and split path.
//
// Same work decomposition, MFMA layout and numerics as attn_fwd.hip; what
// differs is how a 32-key chunk reaches LDS. Loads are ordinary 16-byte
// vector loads into registers, issued as soon as the previous chunk has been
// moved from registers into LDS, so each wave keeps one chunk in flight while
// it computes the chunk before it out of LDS. Two kernels:
//
//  * attn_fwd_pagerows (the vLLM NHD cell of 8 KV heads, work-groups whose
//    8 waves are the 8 heads of the same keys): the work-group loads whole
//    slot rows (every cache line by exactly one wave) into a shared LDS
//    chunk buffer, one barrier per chunk; its QK products are integer (the
//    int8 K bytes against three int8 digits of the scaled query, QInt8 in
//    attn_device.h), so K is never converted;
//  * attn_fwd_staged (any other cell cache): each wave loads its own head's
//    cells in row order (lane (t, c) reads 16-byte piece c of key t, so one
//    instruction covers 8 whole 128-byte rows) into its own LDS slot.
//
// Measured on MI355X with config 2's cache (8 KV heads, pages of 16 keys,
// shuffled pages, 2.2 GB) in a read-only loop: direct-to-LDS loads with one
// 32-key chunk in flight per wave reach 5.2 TB/s, the register-staged row
// loads 6.0 TB/s; two chunks in flight per wave are slower with either.
// The page-row kernel runs config 2 at 364 us (the per-wave staged kernel
// 396 us: its waves read cache lines shared with the neighbouring head and
// re-fetch them when they drift apart).

#include "attn_device.h"

namespace pa {
namespace {

// One 32-key chunk of one KV head in row order, as the lane loaded it:
// k[2 sub + h] / v[2 sub + h] = piece c of key 16 sub + 8 h + t; s = the
// lane's scale (lanes 0..31: K scales of keys 0..31, 32..63: V scales).
struct Staged {
  u32x4 k[4];
  u32x4 v[4];
  float s;
};

// Per-lane source offset within a 16-key group of one page for the unit's
// KV head: piece c of the K row of key t (key 8 + t and the V row are at
// uniform distances from it), and the lane's scale.
struct StageOffsets {
  uint32_t k, s;
};

__device__ __forceinline__ StageOffsets stage_offsets(const AttnParams& p, int kvh, int lane) {
  const uint32_t t = lane >> 3, c = lane & 7;
  const uint32_t head = static_cast<uint32_t>(kvh) * p.cell_head;
  StageOffsets o;
  o.k = t * p.cell_slot + head + 16u * c + p.cell_off[0];
  o.s = static_cast<uint32_t>(lane & 15) * p.cell_slot + head +
        (lane < 32 ? p.cell_off[2] : p.cell_off[3]);
  return o;
}

// Pages and first slots of the two 16-key groups of the chunk starting at
// key c of unit U (scalar loads of the block table; a group outside the
// unit's keys reads page 0 and is masked by the consumer).
struct ChunkPages {
  int32_t page[2], slot0[2];
};

__device__ __forceinline__ ChunkPages chunk_pages(const AttnParams& p, const Unit& U, int c) {
  // The unit is wave-uniform; saying so makes the block-table reads scalar
  // loads (lgkmcnt), which never wait for the chunk loads in flight.
  const int req = __builtin_amdgcn_readfirstlane(U.t.req);
  const int ld_lo = __builtin_amdgcn_readfirstlane(U.ld_lo);
  const int ld_hi = __builtin_amdgcn_readfirstlane(U.ld_hi);
  c = __builtin_amdgcn_readfirstlane(c);
  const int64_t bt0 = static_cast<int64_t>(req) * p.bt_stride;
  ChunkPages cp;
#pragma unroll
  for (int sub = 0; sub < 2; ++sub) {
    const int c16 = c + 16 * sub;
    cp.page[sub] = 0;
    cp.slot0[sub] = 0;
    if (c16 < ld_hi && c16 + 16 > ld_lo) {
      const int blk = static_cast<int>(p.bs_div.div(c16));
      cp.slot0[sub] = c16 - blk * static_cast<int>(p.bs_div.d);
      cp.page[sub] = ld_ro(p.block_table, bt0 + blk);
    }
  }
  return cp;
}

// Issues the 17 loads of one chunk: 8 x 16 B of K and V per lane and one
// scale. Every address is inside the cache (see chunk_pages).
__device__ __forceinline__ void stage_load(const AttnParams& p, const ChunkPages& cp,
                                           const StageOffsets& o, int lane, Staged& S) {
  const char* base[2];
#pragma unroll
  for (int sub = 0; sub < 2; ++sub)
    base[sub] = p.cell_base +
                static_cast<uint64_t>(static_cast<uint32_t>(cp.page[sub])) * p.cell_block +
                static_cast<uint32_t>(cp.slot0[sub]) * p.cell_slot;
  const uint32_t row8 = 8u * p.cell_slot;                  // key t -> key 8 + t
  const int64_t kv = static_cast<int64_t>(p.cell_off[1]) - p.cell_off[0];  // K row -> V row
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const char* a = base[i >> 1] + o.k + ((i & 1) ? row8 : 0u);
    S.k[i] = *reinterpret_cast<const u32x4_a4*>(a);
    S.v[i] = *reinterpret_cast<const u32x4_a4*>(a + kv);
  }
  S.s = *reinterpret_cast<const float*>(((lane >> 4) & 1 ? base[1] : base[0]) + o.s);
}

// Writes a staged chunk into the wave's slot in the layout read_offsets
// reads: key row r at 128 r, its 16-byte piece c at position c ^ (r & 7); the
// scales at kSlotScale + 4 lane (K scales of keys 0..31, then V scales).
__device__ __forceinline__ void stage_write(char* slot, int lane, const Staged& S) {
  const int t = lane >> 3, c = lane & 7;
  const int pos = 16 * (c ^ t);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int key = 8 * i + t;  // 16 sub + 8 h + t with i = 2 sub + h
    *reinterpret_cast<u32x4*>(slot + kSlotK + 128 * key + pos) = S.k[i];
    *reinterpret_cast<u32x4*>(slot + kSlotV + 128 * key + pos) = S.v[i];
  }
  *reinterpret_cast<float*>(slot + kSlotScale + 4 * lane) = S.s;
}

// The chunk's MFMA operands out of the slot (plain LDS loads: the compiler
// orders them after the slot write and waits for them where they are used).
__device__ __forceinline__ void slot_read(const char* slot, const ReadOffsets& o, Chunk& ch) {
#pragma unroll
  for (int sub = 0; sub < 2; ++sub) {
    ch.k[sub][0] = *reinterpret_cast<const u32x4*>(slot + o.k[0] + 2048 * sub);
    ch.k[sub][1] = *reinterpret_cast<const u32x4*>(slot + o.k[1] + 2048 * sub);
  }
#pragma unroll
  for (int e = 0; e < 8; ++e)
    ch.v[e] = *reinterpret_cast<const u32x2*>(slot + o.v[e & 3] + 2048 * (e >> 2));
  ch.sc = *reinterpret_cast<const float*>(slot + o.s);
}

__device__ __forceinline__ int uni(int x) { return __builtin_amdgcn_readfirstlane(x); }

// Every field of a unit is wave-uniform; stating it lets the compiler keep
// them in scalar registers and branch on them without exec masks.
__device__ __forceinline__ void make_uniform(Unit& U) {
  U.t.req = uni(U.t.req);
  U.t.tok_begin = uni(U.t.tok_begin);
  U.t.num_tok = uni(U.t.num_tok);
  U.t.q_len = uni(U.t.q_len);
  U.t.seq_len = uni(U.t.seq_len);
  U.t.q_start = uni(U.t.q_start);
  U.s = uni(U.s);
  U.live = uni(U.live);
  U.kvh = uni(U.kvh);
  U.rg = uni(U.rg);
  U.rows = uni(U.rows);
  U.row0 = uni(U.row0);
  U.has_rows = uni(U.has_rows ? 1 : 0) != 0;
  U.ld_lo = uni(U.ld_lo);
  U.ld_hi = uni(U.ld_hi);
  U.c_begin = uni(U.c_begin);
  U.n_chunks = uni(U.n_chunks);
  U.w_lo_max = uni(U.w_lo_max);
  U.w_hi_min = uni(U.w_hi_min);
}

template <bool kWindow, bool kStream>
__device__ __forceinline__ bool next_live_unit(const AttnParams& p, Work<kWindow, kStream>& work,
                                               int lane, Unit& U, Lanes& L) {
  while (work.next(p, lane, U)) {
    make_uniform(U);
    if (!U.has_rows) continue;
    L = unit_lanes<kWindow>(p, U, lane);
    if (U.n_chunks == 0) {  // no key of these rows in this split
      State empty;
      state_reset(empty);
      epilogue(p, U, L, empty);
      continue;
    }
    return true;
  }
  return false;
}

template <bool kWindow, bool kStream, bool kF16Q>
__global__ __launch_bounds__(kFwdWaves * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attn_fwd_staged(const AttnParams p_arg) {
  __shared__ __attribute__((aligned(16))) char lds_all[kFwdWaves * kSlotBytes];
  const int lane = threadIdx.x & 63;
  const AttnParams p = params_in_registers(p_arg, lane);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  char* slot = lds_all + wave * kSlotBytes;
  const ReadOffsets ro = read_offsets(lane);
  const float scl = scale_factor(lane & 15, p.scale_log2);

  Work<kWindow, kStream> work;
  work.init(p, lane);
  Unit U;
  Lanes L;
  int realign = 0;
  while (next_live_unit(p, work, lane, U, L)) {
    const StageOffsets so = stage_offsets(p, U.kvh, lane);
    Staged S;
    ChunkPages cp = chunk_pages(p, U, U.c_begin);
    stage_load(p, cp, so, lane, S);
    bf16x8 qb[4], qlo[4];
    load_q<kF16Q>(p, L, qb, qlo);
    if (U.n_chunks > 1) cp = chunk_pages(p, U, U.c_begin + kChunkTokens);
    State st;
    state_reset(st);
    for (int k = 0; k < U.n_chunks; ++k) {
      // Chunk k is in S: move it to the slot, start chunk k + 1, look up the
      // pages of chunk k + 2, then compute chunk k from the slot.
      stage_write(slot, lane, S);
      if (k + 1 < U.n_chunks) {
        stage_load(p, cp, so, lane, S);
        if (k + 2 < U.n_chunks) cp = chunk_pages(p, U, U.c_begin + kChunkTokens * (k + 2));
      }
      Chunk ch;
      slot_read(slot, ro, ch);
      compute_chunk<kF16Q>(U, L, U.c_begin + kChunkTokens * k, ch, qb, qlo, scl, st);
      // Re-align the work-group's waves now and then (they read adjacent
      // cells whose shared cache lines are fetched once while the waves stay
      // close). A wave that has finished no longer holds the others.
      if (++realign == kRealignChunks) {
        realign = 0;
        __builtin_amdgcn_s_barrier();
      }
    }
    epilogue(p, U, L, st);
  }
}


// ---------------------------------------------------------------------------
// Page-row kernel: the vLLM NHD cell cache with 8 KV heads (a slot row is the
// 8 heads' 264-byte cells, 2112 contiguous bytes, so a 16-key group of a page
// is 33,792 contiguous bytes) and work-groups whose 8 waves are the 8 KV
// heads of the same keys. The work-group loads each 32-key chunk as whole
// slot rows: its 512 lanes split the chunk's 67,584 bytes into 16-byte
// pieces (eight per lane, plus one dword), so every cache line is fetched by
// exactly one wave and no line is shared between waves that may drift
// apart. The rows land in a work-group-shared LDS chunk buffer (two
// buffers, one being written while the other is read; rows padded to
// kRowPad bytes so the head-strided operand reads spread over the banks)
// and each wave computes its own head from it. One barrier per chunk.
#ifdef PA_WAVE_CLOCK
constexpr int kMaxClockWaves = 8192;
#endif
constexpr int kRowBytes = 2112;                      // 8 cells of 264 bytes
constexpr int kRowPad = kRowBytes + 16;              // LDS bytes per key row
constexpr int kRowBuf = kChunkTokens * kRowPad;      // one chunk buffer
constexpr int kGroupBytes = 16 * kRowBytes;          // one 16-key group of a page
constexpr int kPiecesPerGroup = kGroupBytes / 16;    // 2112
constexpr int kRowPieces = kRowBytes / 16;           // 132

// The lane's share of one chunk: pieces L + 512 j (j < 8) of the chunk's
// 4224 16-byte pieces and the dword 65536 + 4 L (the tail, all in key 15 of
// the second group), L = the lane's index in the work-group.
struct RowStaged {
  u32x4 piece[8];
  uint32_t tail;
};

// The loads carry the non-temporal hint: every cache line of the chunk is
// fetched by exactly one wave and never again in the launch (config 2:
// 364.5 -> 350.4 us). The kernels whose waves share lines (neighbouring
// heads' cells, the row groups of a KV head) keep ordinary loads: the hint
// there cost config 4 39.6 -> 63.0 us and config 5 4.56 -> 4.81 ms.
__device__ __forceinline__ void rows_load(const AttnParams& p, const ChunkPages& cp, int L,
                                          RowStaged& S) {
  const char* base[2];
#pragma unroll
  for (int sub = 0; sub < 2; ++sub)
    base[sub] = p.cell_base +
                static_cast<uint64_t>(static_cast<uint32_t>(cp.page[sub])) * p.cell_block +
                static_cast<uint32_t>(cp.slot0[sub]) * static_cast<uint32_t>(kRowBytes);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int i = L + 512 * j;
    const int grp = i >= kPiecesPerGroup ? 1 : 0;  // j < 4: 0; j > 4: 1
    const int w = i - grp * kPiecesPerGroup;
    S.piece[j] = ld_nt<u32x4>((grp ? base[1] : base[0]) + 16 * w);
  }
  S.tail = ld_nt<uint32_t>(base[1] + (65536 - kGroupBytes) + 4 * L);
}

__device__ __forceinline__ void rows_write(char* buf, int L, const RowStaged& S) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int i = L + 512 * j;
    const int grp = i >= kPiecesPerGroup ? 1 : 0;
    const int w = i - grp * kPiecesPerGroup;
    const int key = w / kRowPieces;
    const int off = 16 * (w - key * kRowPieces);
    *reinterpret_cast<u32x4*>(buf + (16 * grp + key) * kRowPad + off) = S.piece[j];
  }
  *reinterpret_cast<uint32_t*>(buf + 31 * kRowPad + (65536 - kGroupBytes - 15 * kRowBytes) + 4 * L) =
      S.tail;
}

// The wave's MFMA operands for KV head `head` out of a chunk buffer (the
// per-lane layout of read_chunk; cells are only 4-byte aligned in a row, so
// K is read as 8-byte and V as paired 4-byte words).
__device__ __forceinline__ void rows_read(const char* buf, const AttnParams& p, int head, int lane,
                                          Chunk& ch) {
  const int r16 = lane & 15, g = lane >> 4;
  const char* cell = buf + head * 264;
#pragma unroll
  for (int sub = 0; sub < 2; ++sub) {
    const char* kr = cell + (16 * sub + r16) * kRowPad + p.cell_off[0] + 32 * g;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const u32x2 a = *reinterpret_cast<const u32x2*>(kr + 16 * h);
      const u32x2 b = *reinterpret_cast<const u32x2*>(kr + 16 * h + 8);
      ch.k[sub][h] = (u32x4){a[0], a[1], b[0], b[1]};
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int key = 16 * (e >> 2) + 4 * g + (e & 3);
    const uint32_t* vr = reinterpret_cast<const uint32_t*>(cell + key * kRowPad + p.cell_off[1] + 8 * r16);
    ch.v[e] = (u32x2){vr[0], vr[1]};
  }
  const int e = r16 & 7;
  const int key = 16 * (e >> 2) + 4 * g + (e & 3);
  ch.sc = *reinterpret_cast<const float*>(cell + key * kRowPad + (r16 < 8 ? p.cell_off[2] : p.cell_off[3]));
}

#ifdef PA_WAVE_CLOCK
// Measurement build only (bench_hip/build.py): per wave of the page-row
// kernel, its XCD, start and end time (s_memrealtime, 100 MHz), so the
// benchmark can report the finishing-time spread by XCD.
__device__ uint64_t wave_clock[kMaxClockWaves * 3];
// The XCD a wave runs on: hardware register XCC_ID, bits [3:0].
__device__ __forceinline__ uint32_t xcc_id() {
  return static_cast<uint32_t>(__builtin_amdgcn_s_getreg((3 << 11) | 20)) & 0xf;
}
#endif

template <bool kWindow, bool kStream, bool kF16Q>
__global__ __launch_bounds__(kFwdWaves * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attn_fwd_pagerows(const AttnParams p) {
  __shared__ __attribute__((aligned(16))) char lds_rows[2 * kRowBuf];
#ifdef PA_WAVE_CLOCK
  const uint64_t clock_start = __builtin_amdgcn_s_memrealtime();
#endif
  const int lane = threadIdx.x & 63;
  const int L = threadIdx.x;
  const float scl = scale_factor(lane & 15, p.scale_log2);
  Work<kWindow, kStream> work;
  work.template init<false>(p, lane);
  Unit U;
  Lanes Ls;
  int it = 0;  // chunks processed by the work-group (buffer parity)
  // Every wave of the work-group walks the same units (the 8 KV heads of the
  // same keys), so they all meet the same barriers.
  while (next_live_unit(p, work, lane, U, Ls)) {
    RowStaged S;
    ChunkPages cp = chunk_pages(p, U, U.c_begin);
    rows_load(p, cp, L, S);
    QInt8 qd;
    load_q_int8<kF16Q>(p, Ls, qd);
    if (U.n_chunks > 1) cp = chunk_pages(p, U, U.c_begin + kChunkTokens);
    State st;
    state_reset(st);
    for (int k = 0; k < U.n_chunks; ++k, ++it) {
      char* buf = lds_rows + (it & 1) * kRowBuf;
      // The buffer was last read two chunks ago; every wave has passed the
      // barrier after that read, so it may be overwritten.
      rows_write(buf, L, S);
      if (k + 1 < U.n_chunks) {
        rows_load(p, cp, L, S);
        if (k + 2 < U.n_chunks) cp = chunk_pages(p, U, U.c_begin + kChunkTokens * (k + 2));
      }
      __syncthreads();  // the chunk's rows are in the buffer
      Chunk ch;
      rows_read(buf, p, U.kvh, lane, ch);
      compute_chunk(U, Ls, U.c_begin + kChunkTokens * k, ch, qd, scl, st);
    }
    epilogue(p, U, Ls, st);
  }
#ifdef PA_WAVE_CLOCK
  const int w = static_cast<int>(blockIdx.x) * kFwdWaves + (static_cast<int>(threadIdx.x) >> 6);
  if (lane == 0 && w < kMaxClockWaves) {
    wave_clock[3 * w] = xcc_id();
    wave_clock[3 * w + 1] = clock_start;
    wave_clock[3 * w + 2] = __builtin_amdgcn_s_memrealtime();
  }
#endif
}
}  // namespace

hipError_t launch_staged_kernel(const AttnParams& p, dim3 grid, bool windowed, bool q_f16,
                                hipStream_t stream) {
  const bool st = p.num_splits > 1;
  if (p.page_rows) {
#define PA_LAUNCH(W, St, F) \
  hipLaunchKernelGGL((attn_fwd_pagerows<W, St, F>), grid, dim3(kFwdWaves * 64), 0, stream, p)
    if (windowed) {
      if (st) { if (q_f16) PA_LAUNCH(true, true, true); else PA_LAUNCH(true, true, false); }
      else { if (q_f16) PA_LAUNCH(true, false, true); else PA_LAUNCH(true, false, false); }
    } else {
      if (st) { if (q_f16) PA_LAUNCH(false, true, true); else PA_LAUNCH(false, true, false); }
      else { if (q_f16) PA_LAUNCH(false, false, true); else PA_LAUNCH(false, false, false); }
    }
#undef PA_LAUNCH
    return hipGetLastError();
  }
#define PA_LAUNCH(W, St, F) \
  hipLaunchKernelGGL((attn_fwd_staged<W, St, F>), grid, dim3(kFwdWaves * 64), 0, stream, p)
  if (windowed) {
    if (st) { if (q_f16) PA_LAUNCH(true, true, true); else PA_LAUNCH(true, true, false); }
    else { if (q_f16) PA_LAUNCH(true, false, true); else PA_LAUNCH(true, false, false); }
  } else {
    if (st) { if (q_f16) PA_LAUNCH(false, true, true); else PA_LAUNCH(false, true, false); }
    else { if (q_f16) PA_LAUNCH(false, false, true); else PA_LAUNCH(false, false, false); }
  }
#undef PA_LAUNCH
  return hipGetLastError();
}

}  // namespace pa

#ifdef PA_WAVE_CLOCK
// Copies the last page-row launch's wave clock (XCD, start, end per wave;
// waves of work-groups beyond the grid hold stale values) to host memory.
extern "C" int32_t pth_attn_debug_wave_clock(uint64_t* dst, int64_t waves) {
  const int64_t n = waves < pa::kMaxClockWaves ? waves : pa::kMaxClockWaves;
  return hipMemcpyFromSymbol(dst, HIP_SYMBOL(pa::wave_clock), n * 3 * sizeof(uint64_t)) ==
                 hipSuccess
             ? 0
             : -1;
}
#endif
