// Paged attention of many query rows per sequence (prefill, chunked prefill) on the matrix
// cores, gfx950: bf16 or fp16 (DT), head_dim 128, page size 16, Hq / Hkv = G in {1, 2, 4, 8}.
//
// Work item (one workgroup of NW = 8 waves, or 4 when the sequences have few rows): one kv head
// and 32 NW / G consecutive query positions of one sequence, i.e. 32 NW (position, q head) rows
// that share the kv head's keys: row r is position s0 + r / G, head h * G + r % G. Wave w owns
// rows 32 w .. 32 w + 31 (two 16-row MFMA blocks); two waves per SIMD. The keys are walked in
// 64-token tiles (four pages): K and V come from the pool into registers a tile ahead (buffer
// loads, no branch), then into LDS (16-byte stores, double buffered) in the middle of the tile
// before theirs, one barrier per tile. With eight waves a tile is staged once for 256 rows.
// Both tiles are [d][64 tokens], eight 16-byte units per row, unpadded and swizzled:
//   K: unit u (tokens 8 u .. 8 u + 7) at u ^ ((d / 4) ^ 2 (d % 4)) % 8;
//   V: unit 4 c + j holds tokens 32 c + 4 j .. + 3 then 32 c + 16 + 4 j .. + 3 (the order of the
//      P operand's k slots below, so one 16-byte read is a whole B operand), at unit
//      (4 c + j) ^ sv(d), sv(d) = (d & 1) | 4 ((d / 2) & 1) | 2 ((d / 8) & 1).
// The swizzles follow the bank rules measured on gfx950 (SQ_LDS_BANK_CONFLICT of access
// patterns replayed alone): ds_write_b128 serves lanes 8 k .. 8 k + 7 together over 32
// four-byte banks; ds_read_b128 serves 16 lanes together over 64 banks, in the lane groups
// {0-3, 12-15, 20-23, 24-27} and {4-11, 16-19, 28-31} and the same plus 32. Under them the K and
// V stores, the transposing K reads and the 16-byte V reads are conflict-free. (Eight-byte V
// reads in the K layout were conflict-free one by one, but the compiler pairs those of blocks nb
// and nb + 2 into ds_read2st64_b64, whose two halves per lane share a bank: 8 conflict cycles.)
// Per tile each wave runs
//   S^T = K . Q^T   v_mfma_f32_16x16x32_{bf16,f16}: A = K^T operands built by ds_read_b64_tr_b16
//                   (within each 16-lane group the eight-byte reads of the lanes form a 16 x 4
//                   matrix, and lane i receives elements (4 k + i / 4, i % 4), k < 4; so lane r
//                   of group g reads the four tokens 16 m + 4 (r % 4) .. of K row d0 + r / 4 and
//                   lane i ends with K[token 16 m + i][d0 .. d0 + 3]; two reads, d0 and d0 + 4,
//                   make an operand), B = the wave's q rows (registers, loaded once). Lane l then
//                   holds the scores of row l % 16 for tokens 16 m + 4 (l / 16) + j (m < 4,
//                   j < 4) of the tile.
//   online softmax  per row in fp32, base 2 with the scale folded in; a row's 64 scores sit
//                   in four lanes (l, l ^ 16, l ^ 32, l ^ 48), reduced by two lane swaps.
//   O += P . V      the probabilities are the A operand straight from the score registers
//                   (rounded to DT): k slot 8 (l / 16) + j of 32-token chunk c is token
//                   32 c + 4 (l / 16) + j for j < 4 and 32 c + 16 + 4 (l / 16) + j - 4 after,
//                   and the B operand is V unit 4 c + l / 16 of row 16 nb + l % 16 (one 16-byte
//                   LDS read), so both sides of every MFMA sum the same 32 tokens. O (16 rows x
//                   128 per block) stays in 8 accumulator blocks; lane l holds rows 4 (l / 16) + j,
//                   column l % 16.
// Keys a row may not see (past its causal limit or the sequence's length, on a page whose
// block-table id is outside the pool) score -inf; their V words are zeros from the loads.
//
// Work list: sequence-major, then kv head, then position tile (the last tiles of a sequence,
// which see the most keys when causal, first). A 1-D grid is dispatched round-robin over the 8
// XCDs (workgroup i runs on XCD i % 8); the list is cut into 8 contiguous runs and XCD x takes
// run x in order, so the ~64 workgroups resident on one XCD are the position tiles of one
// (sequence, kv head) and read its K / V through that XCD's L2 once between them.
#include <algorithm>

#include "attn_tiles.h"
#include "pia_internal.h"

namespace pia {
namespace {

using tile::f32x4_t;

constexpr int PF_D = 128, PF_P = 16;
constexpr int PF_RB = 2;              // 16-row MFMA blocks per wave
constexpr int PF_WROWS = 16 * PF_RB;  // (position, head) rows per wave
constexpr int PF_KT = 64;             // keys per tile: four pages
constexpr int PF_MAX_SEQS = 1024;     // sequences per launch (tile prefix in LDS)
constexpr int PF_V_AHEAD = 4;         // V operand reads in flight ahead of the P . V products
// word 3 of a raw (stride 0) buffer descriptor on gfx9 parts; a load at or past the descriptor's
// byte count returns zeros
constexpr int PF_RSRC_WORD3 = 0x00020000;

// lazy rescaling threshold (log2 units): a row's exponentials are taken against a reference
// that trails its true max by at most this much, so probabilities stay <= 2^8
constexpr float PF_RESCALE = 8.0f;

template <int G, int NW, int DT>
__global__ __launch_bounds__(64 * NW, 8 / NW) void paged_prefill_mfma(
    uint16_t* __restrict__ out, const uint16_t* __restrict__ q,
    const uint16_t* __restrict__ kpool, const uint16_t* __restrict__ vpool,
    const int32_t* __restrict__ bt, int64_t bt_stride, const int32_t* __restrict__ kv_lens,
    const int32_t* __restrict__ cu_q, const int32_t* __restrict__ offsets, int B, int Hkv,
    int64_t num_pages, float scale_log2) {
  constexpr int D = PF_D, P = PF_P, TILE = D * P;
  constexpr int NT = 64 * NW;                 // threads per workgroup
  constexpr int PPT = PF_WROWS * NW / G;  // query positions per work item
  constexpr int RB = PF_RB;
  constexpr int XCDS = 8;
  __shared__ __align__(16) uint16_t ks[2][PF_D * PF_KT];
  __shared__ __align__(16) uint16_t vs[2][PF_D * PF_KT];
  __shared__ int tile_pref[PF_MAX_SEQS + 1];
  __shared__ int wsum[NW];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int Hq = Hkv * G;
  const int64_t q_row = int64_t(Hq) * D;  // elements between query positions

  // work items per sequence (ceil(rows / PPT)) and their prefix, scanned NT sequences at a time
  if (tid == 0) tile_pref[0] = 0;
  int carry = 0;
  for (int c0 = 0; c0 < B; c0 += NT) {
    const int i = c0 + tid;
    const int n = i < B ? (cu_q ? cu_q[i + 1] - cu_q[i] : 1) : 0;
    const int t = n > 0 ? (n + PPT - 1) / PPT : 0;
    int incl = t;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(incl, o, 64);
      if (lane >= o) incl += y;
    }
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    int base = carry;
    for (int x = 0; x < wave; ++x) base += wsum[x];
    if (i < B) tile_pref[i + 1] = base + incl;
#pragma unroll
    for (int x = 0; x < NW; ++x) carry += wsum[x];
    __syncthreads();
  }
  // this workgroup's item: XCD x = blockIdx % 8 runs items [x * run, (x + 1) * run) in order
  const int64_t items = int64_t(carry) * Hkv;
  const int64_t run = (items + XCDS - 1) / XCDS;
  const int64_t k = blockIdx.x / XCDS;
  const int64_t item = (blockIdx.x % XCDS) * run + k;
  if (k >= run || item >= items) return;
  int lo = 0, hi = B - 1;  // the sequence holding the item: Hkv * tile_pref[b] <= item
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (int64_t(tile_pref[mid]) * Hkv <= item) lo = mid; else hi = mid - 1;
  }
  const int b = lo;
  const int nt_b = tile_pref[b + 1] - tile_pref[b];
  const int rem = int(item - int64_t(tile_pref[b]) * Hkv);
  const int h = rem / nt_b;
  const int s0 = (nt_b - 1 - rem % nt_b) * PPT;
  const int64_t row0 = cu_q ? int64_t(cu_q[b]) : int64_t(b);
  const int n_b = cu_q ? cu_q[b + 1] - cu_q[b] : 1;
  int kv_len = kv_lens[b];
  kv_len = kv_len < 0 ? 0 : (int64_t(kv_len) > bt_stride * P ? int(bt_stride * P) : kv_len);
  const int off = offsets ? offsets[b] : 0;
  const int s_last = min(s0 + PPT, n_b) - 1;
  int kmax = kv_len;
  if (offsets) kmax = max(0, min(kmax, off + s_last + 1));
  const int npages = (kv_len + P - 1) / P;
  const int nkt = (kmax + PF_KT - 1) / PF_KT;
  const int32_t* btb = bt + int64_t(b) * bt_stride;

  // this lane's score rows: 32 wave + 16 rb + l % 16 (rb < RB) and their q operands,
  // d = 32 kc + 8 (l / 16) .. + 7
  const int g4 = lane >> 4, n16 = lane & 15;
  int lim_r[RB];
  uint4 qreg[RB][4];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int r = 32 * wave + 16 * rb + n16;
    const int sr = s0 + r / G;
    const bool ok = sr < n_b;
    lim_r[rb] = !ok ? 0 : (offsets ? min(kv_len, off + sr + 1) : kv_len);
    const uint16_t* qp = q + (row0 + (ok ? sr : 0)) * q_row + int64_t(h * G + r % G) * D;
#pragma unroll
    for (int kc = 0; kc < 4; ++kc)
      qreg[rb][kc] = ok ? *reinterpret_cast<const uint4*>(qp + 32 * kc + 8 * g4)
                        : make_uint4(0u, 0u, 0u, 0u);
  }
  // every valid row of the item sees at least the keys below lim_min (the first row's limit)
  const int lim_min = offsets ? max(0, min(kv_len, off + s0 + 1)) : kv_len;

  // tile loads: with four waves, thread t moves row d = t / 2, tokens 8 (t % 2) .. + 7 of each of
  // the tile's four (page, head) K and V tiles; with eight, wave w moves pages 2 (w % 2) and
  // 2 (w % 2) + 1 (the page pair is uniform in the wave), row d = 32 (w / 2) + l / 2, tokens
  // 8 (l % 2) .. + 7. NCP: page pairs per thread, cp0: its first pair.
  constexpr int NCP = NW == 4 ? 2 : 1;
  const int cp0 = NW == 4 ? 0 : (wave & 1);
  const int ld_d = NW == 4 ? tid >> 1 : 32 * (wave >> 1) + (lane >> 1), ld_half = tid & 1;
  const int ld_off = ld_d * P + ld_half * 8;  // the thread's piece inside a (page, head) tile
  // kr[q]: the thread's K piece of its page q (tile page 2 cp0 + q); vu[2 cc + e]: its V unit
  // 4 c + 2 h + e (c = cp0 + cc, h = ld_half), tokens 8 h + 4 e .. + 3 of page 2 c in .x/.y and
  // of page 2 c + 1 in .z/.w, loaded by eight-byte loads straight into place (a unit assembled
  // from two 16-byte loads would need register copies that wait on the loads)
  uint4 kr[2 * NCP], vu[2 * NCP];
  // block-table ids of a tile: lane i < 4 holds page 4 kt + i's id (-1 past the table). They
  // are loaded a tile ahead of the fetch that uses them, with one vector load, so no tile
  // waits on a chain of dependent block-table reads.
  auto bt_of = [&](int kt) -> int {
    const int pi = 4 * kt + lane;
    return (lane < 4 && pi < npages) ? btb[pi] : -1;
  };
  // ld_off + 4, hidden from the compiler so it does not fuse the two V loads into one
  int ld_off4 = ld_off + 4;
  asm volatile("" : "+v"(ld_off4));
  // Pages go through buffer descriptors (an id outside the pool gets an empty one, whose loads
  // return zeros), so the fetch has no branch: the wait for the block-table load issued before it
  // then counts exactly the fetch's loads after it instead of waiting for all of them.
  const uint32_t np32 = num_pages > 0x7fffffff ? 0x7fffffffu : uint32_t(num_pages);
  auto page_rsrc = [&](const uint16_t* pool, int id) {
    const bool ok = uint32_t(id) < np32;
    const int64_t tile_off = (int64_t(ok ? id : 0) * Hkv + h) * TILE;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(pool + tile_off), 0,
                                             ok ? TILE * 2 : 0, PF_RSRC_WORD3);
  };
  auto fetch = [&](int bt4) {
#pragma unroll
    for (int q = 0; q < 2 * NCP; ++q) {
      const int id = __builtin_amdgcn_readlane(bt4, 2 * cp0 + q);
      const __amdgpu_buffer_rsrc_t kres = page_rsrc(kpool, id), vres = page_rsrc(vpool, id);
      kr[q] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(kres, 2 * ld_off,
                                                                               0, 0));
      const auto l0 = __builtin_amdgcn_raw_buffer_load_b64(vres, 2 * ld_off, 0, 0);
      const auto l1 = __builtin_amdgcn_raw_buffer_load_b64(vres, 2 * ld_off4, 0, 0);
      const uint2 v0 = make_uint2(l0[0], l0[1]), v1 = make_uint2(l1[0], l1[1]);
      const int i = q;  // the thread's page q: V units 2 (q / 2), 2 (q / 2) + 1, half q % 2
      uint4& u0 = vu[2 * (i >> 1)];
      uint4& u1 = vu[2 * (i >> 1) + 1];
      if (i & 1) {
        u0.z = v0.x; u0.w = v0.y; u1.z = v1.x; u1.w = v1.y;
      } else {
        u0.x = v0.x; u0.y = v0.y; u1.x = v1.x; u1.y = v1.y;
      }
    }
  };
  // Swizzled LDS offsets, as per-lane bases XORed with compile-time terms (the unit index split
  // into its bits): the K store of piece i lands at st_base ^ 16 i; the K operand read
  // (kc, hi, mb) at (k_base[hi] ^ 16 mb) + 2048 kc; the V stores (c, e) at v_st ^ (32 c + 8 e);
  // the V operand read (c, nb) at (v_rd ^ 32 c) + 1024 nb.
  int st_base, k_base[2], v_st, v_rd;
  {
    const int f = ((ld_d >> 2) ^ ((ld_d & 3) << 1)) & 7;
    st_base = (ld_d * PF_KT + 8 * (ld_half ^ (f & 1))) | (16 * (f >> 1));
#pragma unroll
    for (int hi = 0; hi < 2; ++hi) {
      const int fk = ((2 * g4 + hi) ^ ((n16 >> 2) << 1)) & 7;
      const int row = 8 * g4 + 4 * hi + (n16 >> 2);
      k_base[hi] = (row * PF_KT + 4 * (n16 & 1) + 8 * (((n16 >> 1) & 1) ^ (fk & 1))) |
                   (16 * (fk >> 1));
    }
    auto sv = [](int d) { return (d & 1) | ((d << 1) & 4) | ((d >> 2) & 2); };
    v_st = ld_d * PF_KT + 8 * ((2 * ld_half) ^ sv(ld_d));
    v_rd = n16 * PF_KT + 8 * (g4 ^ sv(n16));  // sv(16 nb + n16) = sv(n16)
  }
  // tokens past kv_len on the sequence's last page: their V words are zeroed before they reach
  // LDS (stale pool memory may hold non-finite values, and p = 0 times inf is not 0)
  const int tail = kv_len - P * (npages - 1);  // keys on the last page, 1..16
  auto stage = [&](int buf, int kt) {
#pragma unroll
    for (int i = 0; i < 2 * NCP; ++i) {  // the thread's page i, tile page 2 cp0 + i
      *reinterpret_cast<uint4*>(&ks[buf][st_base ^ (16 * (2 * cp0 + i))]) = kr[i];
      if (4 * kt + 2 * cp0 + i == npages - 1 && tail < P) {  // uniform
        const int nv = tail - 8 * ld_half;
        uint4& u0 = vu[2 * (i >> 1)];
        uint4& u1 = vu[2 * (i >> 1) + 1];
        if (i & 1) {
          u0.z = tile::mask_pair(u0.z, 0, nv); u0.w = tile::mask_pair(u0.w, 2, nv);
          u1.z = tile::mask_pair(u1.z, 4, nv); u1.w = tile::mask_pair(u1.w, 6, nv);
        } else {
          u0.x = tile::mask_pair(u0.x, 0, nv); u0.y = tile::mask_pair(u0.y, 2, nv);
          u1.x = tile::mask_pair(u1.x, 4, nv); u1.y = tile::mask_pair(u1.y, 6, nv);
        }
      }
    }
#pragma unroll
    for (int cc = 0; cc < NCP; ++cc) {
      const int c = cp0 + cc;
      *reinterpret_cast<uint4*>(&vs[buf][v_st ^ (32 * c)]) = vu[2 * cc];
      *reinterpret_cast<uint4*>(&vs[buf][v_st ^ (32 * c + 8)]) = vu[2 * cc + 1];
    }
  };
  // V operand i = 8 c + nb of a tile: unit 4 c + l / 16 of row 16 nb + l % 16
  auto vread = [&](int buf, int i) {
    return *reinterpret_cast<const uint4*>(&vs[buf][(v_rd ^ (32 * (i >> 3))) + 1024 * (i & 7)]);
  };
  // pages of a tile that hold keys: bit i for page i (lane i < 4 holds page i's id)
  auto page_mask = [&](int bt4) {
    return int(__ballot(lane < 4 && uint32_t(bt4) < np32) & 0xFull);
  };

  // m[rb]: the row's running max in raw score units, the reference point of its exponentials.
  // It only moves when a tile's max exceeds it by more than PF_RESCALE / scale_log2 (lazy
  // rescaling: probabilities up to 2^PF_RESCALE in between, exact after the final division).
  // acc[rb][8] is the row's unnormalised output in the MFMA layout (rows 4 g4 + j, column
  // l % 16); lsum[rb] is its softmax denominator, summed by the matrix cores against a column
  // of ones, so it sits in the same layout and is rescaled with the accumulators.
  float m[RB];
  f32x4_t acc[RB][8], lsum[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    m[rb] = -INFINITY;
    lsum[rb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) acc[rb][nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  const uint4 ones = tile::ones16<DT>();

  // Tile 0 is staged before the loop; tile kt + 1 is staged in the middle of tile kt (after its
  // softmax, before its P . V), from registers fetched a tile earlier, and the fetch of tile
  // kt + 2 follows at once. The barrier at each tile's end publishes the next tile and frees
  // the buffer the tile read. The fetches run unconditionally (past the last tile they load
  // data no stage uses): with no branch around them, the wait for the block-table load issued
  // before a fetch counts exactly the fetch's loads instead of waiting for all of them.
  int bt_cur = bt_of(0), bt_nxt = bt_of(1), bt_far = bt_of(2);
  fetch(bt_cur);
  stage(0, 0);
  fetch(bt_nxt);
  __syncthreads();
  for (int kt = 0; kt < nkt; ++kt) {
    const int buf = kt & 1;
    const int pmask = page_mask(bt_cur);
    // a tile every valid row sees whole (interior of the causal triangle, all pages valid)
    const bool full = pmask == 0xF && (kt + 1) * PF_KT <= lim_min;
    const int bt_next_far = bt_of(kt + 3);

    // S^T for the wave's rows: 4 token blocks (one per page) x 4 d chunks, each K operand
    // serving both row blocks; d chunk outermost, so consecutive products of one accumulator
    // are 4 RB MFMAs apart (a product that reads the result of the one just issued waits for
    // it to drain)
    f32x4_t sc[RB][4];
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) {
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const uint2 lo = tile::read_tr16(&ks[buf][(k_base[0] ^ (16 * mb)) + 2048 * kc]);
        const uint2 hi = tile::read_tr16(&ks[buf][(k_base[1] ^ (16 * mb)) + 2048 * kc]);
        const uint4 a = make_uint4(lo.x, lo.y, hi.x, hi.y);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
          sc[rb][mb] = tile::mfma16<DT>(a, qreg[rb][kc],
                                       kc == 0 ? f32x4_t{0.f, 0.f, 0.f, 0.f} : sc[rb][mb]);
      }
    }
    uint4 pk[RB][2];
    bool moved = false;
    float alpha[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      // on boundary tiles, keys the row may not see (tokens 64 kt + 16 mb + 4 g4 + j) -> -inf
      if (!full) {
        // token 64 kt + 16 mb + 4 g4 + j is visible to the row when 16 mb + j < rel (one
        // per-lane value and immediates: written with the token index per element, the
        // compiler computed all sixteen indices ahead of the branch, on every tile)
        const int rel = lim_r[rb] - (kt * PF_KT + 4 * g4);
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (!(16 * mb + j < rel && ((pmask >> mb) & 1))) sc[rb][mb][j] = -INFINITY;
      }
      // the row max with IEEE 754-2019 maximum (a NaN score makes it NaN, and the row's output
      // NaN, as the reference's softmax gives): v_maximum3_f32, no quieting of the scores
      float mx = -INFINITY;
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
        mx = __builtin_elementwise_maximum(
            mx, __builtin_elementwise_maximum(
                    __builtin_elementwise_maximum(sc[rb][mb][0], sc[rb][mb][1]),
                    __builtin_elementwise_maximum(sc[rb][mb][2], sc[rb][mb][3])));
      mx = tile::maximum_col4(mx);
      // move the reference point only for a large enough rise (or the first keys of the row)
      const float mref = (mx - m[rb]) * scale_log2 > PF_RESCALE ? mx : m[rb];
      alpha[rb] = m[rb] == mref ? 1.f : __builtin_amdgcn_exp2f((m[rb] - mref) * scale_log2);
      moved = moved || m[rb] != mref;
      m[rb] = mref;
      // p = 2^((s - m) * scale_log2); a row with no key yet keeps m = -inf and p = 0
      const float nm = mref == -INFINITY ? 0.f : -mref * scale_log2;
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        float p[2][4];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            p[hh][j] = __builtin_amdgcn_exp2f(fmaf(sc[rb][2 * c + hh][j], scale_log2, nm));
        pk[rb][c] = make_uint4(
            tile::pack16x2<DT>(p[0][0], p[0][1]), tile::pack16x2<DT>(p[0][2], p[0][3]),
            tile::pack16x2<DT>(p[1][0], p[1][1]), tile::pack16x2<DT>(p[1][2], p[1][3]));
      }
    }
    // rescale O and the sums when some row's reference point moved: lane l's accumulator rows
    // are 4 g4 + j of each block; their alpha sits in lane 4 g4 + j
    if (__ballot(moved)) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        float aj[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) aj[j] = __shfl(alpha[rb], 4 * g4 + j, 64);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          lsum[rb][j] *= aj[j];
#pragma unroll
          for (int nb = 0; nb < 8; ++nb) acc[rb][nb][j] *= aj[j];
        }
      }
    }
    stage(buf ^ 1, kt + 1);
    fetch(bt_far);
    // O += P . V over the tile's two 32-token chunks, each V operand serving both row blocks;
    // the sums against a column of ones. Chunk outermost: consecutive products of one
    // accumulator are 8 RB + RB MFMAs apart. The V operands (i = 8 c + nb) are read
    // PF_V_AHEAD products ahead of their use, so the LDS latency hides behind the MFMAs.
    uint4 vq[PF_V_AHEAD];
#pragma unroll
    for (int i = 0; i < PF_V_AHEAD; ++i) vq[i] = vread(buf, i);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int c = i >> 3, nb = i & 7;
      const uint4 vop = vq[i % PF_V_AHEAD];
      if (i + PF_V_AHEAD < 16) vq[i % PF_V_AHEAD] = vread(buf, i + PF_V_AHEAD);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) acc[rb][nb] = tile::mfma16<DT>(pk[rb][c], vop, acc[rb][nb]);
      if (nb == 7) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) lsum[rb] = tile::mfma16<DT>(pk[rb][c], ones, lsum[rb]);
      }
    }
    // keep that order through the machine scheduler (it would sink the reads to their uses):
    // PF_V_AHEAD reads, then one read per RB products, then the rest of the products
    __builtin_amdgcn_sched_group_barrier(0x100, PF_V_AHEAD, 0);
#pragma unroll
    for (int i = 0; i < 16 - PF_V_AHEAD; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, RB, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, RB * (PF_V_AHEAD + 2), 0);
    __syncthreads();
    bt_cur = bt_nxt;
    bt_nxt = bt_far;
    bt_far = bt_next_far;
  }

  // out = O / sum for rows 4 g4 + j of each block
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float lj = lsum[rb][j];
      const int r = 32 * wave + 16 * rb + 4 * g4 + j;
      const int s = s0 + r / G;
      if (s >= n_b) continue;
      uint16_t* o = out + (row0 + s) * q_row + int64_t(h * G + r % G) * D + n16;
      const float inv = lj > 0.f ? 1.f / lj : 0.f;
#pragma unroll
      for (int nb = 0; nb < 8; ++nb)
        o[16 * nb] = DT == PIA_DTYPE_F16 ? f32_to_half(acc[rb][nb][j] * inv)
                                         : f32_to_bf16(acc[rb][nb][j] * inv);
    }
}

}  // namespace

bool prefill_mfma_path(int dtype, int Hq, int Hkv, int D, int P, int num_seqs,
                       int64_t total_q_rows, const int32_t* cu_q, float scale) {
  const int G = Hq / Hkv;
  // scale > 0: the kernel keeps its running max in raw score units
  return (dtype == PIA_DTYPE_BF16 || dtype == PIA_DTYPE_F16) && D == PF_D && P == PF_P &&
         scale > 0.f &&
         (G == 1 || G == 2 || G == 4 || G == 8) && cu_q != nullptr && num_seqs <= PF_MAX_SEQS &&
         total_q_rows >= 4 * int64_t(num_seqs);
}

int launch_prefill_mfma(int dtype, void* out, const void* q, const void* k_pages,
                        const void* v_pages, const int32_t* bt, int64_t bt_stride, const int32_t* kv_lens,
                        const int32_t* cu_q, const int32_t* offsets, int num_seqs,
                        int64_t total_q_rows, int Hq, int Hkv, int64_t num_pages,
                        float scale_log2, hipStream_t s) {
  const int G = Hq / Hkv;
  // eight waves (256 rows per item, one K / V tile staged for all of them) when the sequences
  // average at least half an item, else four (128 rows)
  const bool wide = 2 * total_q_rows >= int64_t(8 * PF_WROWS / G) * num_seqs;
  const int ppt = (wide ? 8 : 4) * PF_WROWS / G;
  // work items: at most ceil(total rows / ppt) + one partial item per sequence
  const int64_t items = (ceil_div(total_q_rows, ppt) + num_seqs) * Hkv;
  const int64_t blocks = ceil_div(items, 8) * 8;
  if (blocks > 0x7fffffff)
    return fail(PIA_EINVAL, "paged_attention: too many query rows for the prefill kernel");
  const dim3 grid{unsigned(blocks), 1u, 1u};
#define PIA_PF(GG, NW)                                                                         \
  hipLaunchKernelGGL((paged_prefill_mfma<GG, NW, DT>), grid, dim3(64 * NW), 0, s,              \
                     reinterpret_cast<uint16_t*>(out), reinterpret_cast<const uint16_t*>(q),   \
                     reinterpret_cast<const uint16_t*>(k_pages),                               \
                     reinterpret_cast<const uint16_t*>(v_pages), bt, bt_stride, kv_lens, cu_q, \
                     offsets, num_seqs, Hkv, num_pages, scale_log2)
#define PIA_PF_G(NW)                  \
  switch (G) {                        \
    case 1: PIA_PF(1, NW); break;     \
    case 2: PIA_PF(2, NW); break;     \
    case 4: PIA_PF(4, NW); break;     \
    default: PIA_PF(8, NW); break;    \
  }
#define PIA_PF_D(NW)                           \
  if (dtype == PIA_DTYPE_F16) {                \
    constexpr int DT = PIA_DTYPE_F16;          \
    PIA_PF_G(NW)                               \
  } else {                                     \
    constexpr int DT = PIA_DTYPE_BF16;         \
    PIA_PF_G(NW)                               \
  }
  if (wide) {
    PIA_PF_D(8);
  } else {
    PIA_PF_D(4);
  }
#undef PIA_PF_D
#undef PIA_PF_G
#undef PIA_PF
  return check_launch("paged_prefill_mfma");
}

}  // namespace pia
