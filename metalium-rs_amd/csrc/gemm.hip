// Matrix products on the gfx950 matrix cores (MFMA).
//
// Reference: Engine::matmul_dram / matmul_dram_bf16 / matmul_dram_batched
// (crates/burn-tt/src/server.rs:178-239) over Session::matmul_dram_as and
// matmul_dram_batched (crates/tt-kernels/src/session.rs:8990, 9415); the routing
// `float_matmul` / `batched_matmul` (crates/burn-tt/src/ops.rs:2833-3052), where
// a transposed operand is a view, not a copy; BF16 products accumulated in F32
// and rounded once (crates/burn-tt/src/ops/rounded.rs:75-120).
//
// MI355X design
//  * One kernel template for both precisions.  BF16 x BF16 runs
//    v_mfma_f32_32x32x16_bf16 (each lane supplies 8 consecutive k of one row
//    of A and one column of B); anything with an F32 operand runs
//    v_mfma_f32_32x32x2f32 in full F32 (BF16 operands widen exactly).
//  * Operand tiles live in LDS as [rows][k] with 128-byte rows (64 BF16 or 32
//    F32 of k) and a 16-byte-chunk XOR swizzle (chunk c of row r stored at
//    c ^ (r & 7)), so the MFMA fragment reads (one 16-byte chunk per lane, 32
//    consecutive rows per half-wave) and the tile writes are conflict-free.
//  * An operand whose k is contiguous in HBM (A as [m, k], a transposed B as
//    [n, k]) is copied chunk by chunk; one whose m/n is contiguous (A
//    transposed, B as [k, n]) is read as 8x8 (BF16) or 4x4 (F32) blocks and
//    transposed in registers before its LDS write.  Transposed operands are
//    never materialised.
//  * Two LDS stages: the next k-tile's global loads are issued before the
//    current tile's MFMAs, written to the other stage after them, one barrier
//    per k-tile.
//  * Tile order is XCD-aware: MI355X deals workgroups round-robin over its 8
//    XCDs (each with its own L2), so consecutive workgroup ids are remapped
//    so that each XCD owns a compact group of output tiles sharing A rows and
//    B columns.
//  * Shapes that are not multiples of the tile take a guarded variant
//    (zero-filled loads, masked stores) of the same kernel.
#include "common.hpp"
#include "tails.hpp"
#include "wave.hpp"

namespace mi {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Element types: uint16_t carries BF16 bits, float is F32.
template <typename T> struct Elt;
template <> struct Elt<uint16_t> { static constexpr int CH = 8; };  // elements per 16-byte chunk
template <> struct Elt<float> { static constexpr int CH = 4; };

__device__ __forceinline__ float to_f32(uint16_t h) { return bf16_bits_to_f32(h); }
__device__ __forceinline__ float to_f32(float f) { return f; }

// Convert one element of the source type S to the MFMA operand type T.
template <typename T, typename S> __device__ __forceinline__ T conv(S v);
template <> __device__ __forceinline__ uint16_t conv<uint16_t, uint16_t>(uint16_t v) { return v; }
template <> __device__ __forceinline__ float conv<float, float>(float v) { return v; }
template <> __device__ __forceinline__ float conv<float, uint16_t>(uint16_t v) { return bf16_bits_to_f32(v); }

// A 16-byte chunk of T.
union Chunk {
  uint4 u;
  uint16_t h[8];
  float f[4];
};

// Load CH consecutive elements of S starting at p and convert to one chunk of T.
template <typename T, typename S>
__device__ __forceinline__ Chunk load_chunk(const S *p) {
  Chunk c;
  if constexpr (sizeof(S) == sizeof(T)) {
    c.u = *reinterpret_cast<const uint4 *>(p);
  } else {  // BF16 source widened to F32: 4 elements = 8 bytes
    uint2 v = *reinterpret_cast<const uint2 *>(p);
    c.f[0] = __uint_as_float(v.x << 16);
    c.f[1] = __uint_as_float(v.x & 0xffff0000u);
    c.f[2] = __uint_as_float(v.y << 16);
    c.f[3] = __uint_as_float(v.y & 0xffff0000u);
  }
  return c;
}

// Guarded form: element e of the chunk read only if e < valid and the chunk is in range.
template <typename T, typename S>
__device__ __forceinline__ Chunk load_chunk_guard(const S *p, int valid) {
  constexpr int CH = Elt<T>::CH;
  Chunk c;
  c.u = make_uint4(0, 0, 0, 0);
#pragma unroll
  for (int e = 0; e < CH; ++e) {
    if (e < valid) {
      if constexpr (sizeof(T) == 2) c.h[e] = conv<T, S>(p[e]);
      else c.f[e] = conv<T, S>(p[e]);
    }
  }
  return c;
}

// Swizzled LDS byte offset of chunk c of row r (128-byte rows).
__device__ __forceinline__ int lds_off(int r, int c) { return r * 128 + ((c ^ (r & 7)) << 4); }

// Per-operand tile loader.  ROWS = tile rows (m or n); the k extent is 128
// bytes of T.  KCONTIG: source element (r, k) at src[r * ld + k]; otherwise at
// src[k * ld + r].
template <typename T, typename S, int ROWS, int NT, bool KCONTIG, bool GUARD>
struct TileLoader {
  static constexpr int CH = Elt<T>::CH;
  static constexpr int BK = 128 / sizeof(T);
  static constexpr int KCH = BK / CH;  // 8 chunks per LDS row
  static_assert(KCH == 8, "128-byte LDS rows");
  // KCONTIG: chunks per thread; else CHxCH blocks per thread (CH chunks each).
  // A thread whose index runs past the tile's last chunk or block idles.
  static constexpr int TOTAL_CHUNKS = ROWS * KCH;
  static constexpr int TOTAL_BLKS = (ROWS / CH) * KCH;
  static constexpr int NCHUNK = (TOTAL_CHUNKS + NT - 1) / NT;
  static constexpr int NBLK = (TOTAL_BLKS + NT - 1) / NT;
  static constexpr bool CHUNK_EVEN = TOTAL_CHUNKS % NT == 0;
  static constexpr bool BLK_EVEN = TOTAL_BLKS % NT == 0;
  static constexpr int NREG = KCONTIG ? NCHUNK : NBLK * CH;
  static_assert(ROWS % CH == 0, "tile rows a multiple of the chunk");
  Chunk reg[NREG];

  // Issue the global loads of the k-tile starting at k0 for tile rows
  // starting at r0.  The chunks stay raw in registers; a transposition (if
  // any) waits for `store`, so the loads' latency overlaps the MFMAs issued
  // between the two calls.
  __device__ __forceinline__ void load(const S *src, int64_t ld, int64_t r0, int64_t k0, int64_t rows_total,
                                       int64_t k_total, int tid) {
    if constexpr (KCONTIG) {
#pragma unroll
      for (int i = 0; i < NCHUNK; ++i) {
        const int q = tid + i * NT;
        if (!CHUNK_EVEN && q >= TOTAL_CHUNKS) break;
        const int r = q / KCH, c = q % KCH;
        const int64_t gr = r0 + r, gk = k0 + c * CH;
        const S *p = src + gr * ld + gk;
        if constexpr (GUARD) {
          int valid = (gr < rows_total) ? static_cast<int>(k_total - gk) : 0;
          valid = valid < 0 ? 0 : (valid > CH ? CH : valid);
          // Vector path only when the whole chunk is in range and aligned.
          if (valid == CH && ((reinterpret_cast<uintptr_t>(p) & (sizeof(S) * CH - 1)) == 0))
            reg[i] = load_chunk<T, S>(p);
          else
            reg[i] = load_chunk_guard<T, S>(p, valid);
        } else {
          reg[i] = load_chunk<T, S>(p);
        }
      }
    } else {
#pragma unroll
      for (int b = 0; b < NBLK; ++b) {
        const int q = tid + b * NT;
        if (!BLK_EVEN && q >= TOTAL_BLKS) break;
        const int kb = q % KCH, rb = q / KCH;
#pragma unroll
        for (int i = 0; i < CH; ++i) {
          const int64_t gk = k0 + kb * CH + i, gr = r0 + rb * CH;
          const S *p = src + gk * ld + gr;
          Chunk &in = reg[b * CH + i];
          if constexpr (GUARD) {
            int valid = (gk < k_total) ? static_cast<int>(rows_total - gr) : 0;
            valid = valid < 0 ? 0 : (valid > CH ? CH : valid);
            if (valid == CH && ((reinterpret_cast<uintptr_t>(p) & (sizeof(S) * CH - 1)) == 0))
              in = load_chunk<T, S>(p);
            else
              in = load_chunk_guard<T, S>(p, valid);
          } else {
            in = load_chunk<T, S>(p);
          }
        }
      }
    }
  }

  // Write the loaded k-tile to LDS (transposing CH x CH blocks of an m/n-
  // contiguous operand so that every LDS row holds k-contiguous chunks).
  __device__ __forceinline__ void store(char *lds, int tid) const {
    if constexpr (KCONTIG) {
#pragma unroll
      for (int i = 0; i < NCHUNK; ++i) {
        const int q = tid + i * NT;
        if (!CHUNK_EVEN && q >= TOTAL_CHUNKS) break;
        const int r = q / KCH, c = q % KCH;
        *reinterpret_cast<uint4 *>(lds + lds_off(r, c)) = reg[i].u;
      }
    } else {
#pragma unroll
      for (int b = 0; b < NBLK; ++b) {
        const int q = tid + b * NT;
        if (!BLK_EVEN && q >= TOTAL_BLKS) break;
        const int kb = q % KCH, rb = q / KCH;
        const Chunk *in = &reg[b * CH];
        // out[j] holds k = 0..CH-1 of row j.
#pragma unroll
        for (int j = 0; j < CH; ++j) {
          Chunk o;
          if constexpr (sizeof(T) == 2) {
#pragma unroll
            for (int m = 0; m < 4; ++m) {
              const uint32_t lo = reinterpret_cast<const uint32_t *>(&in[2 * m].u)[j >> 1];
              const uint32_t hi = reinterpret_cast<const uint32_t *>(&in[2 * m + 1].u)[j >> 1];
              reinterpret_cast<uint32_t *>(&o.u)[m] =
                  (j & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
            }
          } else {
#pragma unroll
            for (int m = 0; m < 4; ++m) o.f[m] = in[m].f[j];
          }
          *reinterpret_cast<uint4 *>(lds + lds_off(rb * CH + j, kb)) = o.u;
        }
      }
    }
  }
};

struct GemmArgs {
  const void *a;
  const void *b;
  void *c;
  int64_t M, N, K;
  int64_t lda, ldb, ldc;
  int64_t sa, sb, sc;  // batch strides in elements (0 = broadcast)
  // Items come in groups: item z = (z / per_group, z % per_group) starts at
  // (z / per_group) * s?2 + (z % per_group) * s? (one group: per_group = batch).
  int64_t per_group;
  int64_t sa2, sb2, sc2;
  int tiles_m, tiles_n;
  int64_t kc;          // split-K: k per slice (blockIdx.z), 0 for none
  // Epilogue of a linear layer (batch 1): C = resid + (A B + bias), each sum
  // rounded in that order; null pointers skip the term.
  const float *bias;   // [N]
  const float *resid;  // [M, N], row pitch ldr
  int64_t ldr;
  // Direct BF16 kernel only: B's own k extent when A's k loop runs over
  // several copies of it (A = [hi | lo] parts of an F32 operand against one
  // B: B's k wraps modulo kb; 0 for none).
  int64_t kb = 0;
  // Direct BF16 kernel only: B's rows are gate|up pairs (32 gate rows, then
  // the 32 up rows of the same outputs, ...), and C receives silu(gate) * up
  // for the N / 2 outputs -- SWIGLU_PARTS: as its BF16 parts ([M, N] BF16: a
  // row's heads, then its remainders); SWIGLU_BF16 / SWIGLU_F32: [M, N / 2]
  // rounded once to BF16, or F32; 0 for a plain product.
  int swiglu = 0;
  QkvTail qkv;  // direct BF16 kernel only: the q|k|v tail instead of C
};

// The epilogue over one 32 x 32 accumulator fragment, whose lane holds column
// `col` at rows row0 + 8 (r / 4) + r % 4: the fragment's 16 residual values
// and its bias are all requested before any result is stored.  The result
// may be the residual itself (an in-place update), so a residual load issued
// after a store the compiler cannot prove disjoint waits for that store; per
// value, that chain made the write-out latency-bound.  Out-of-range values
// (GUARD) are not read.
template <bool GUARD>
__device__ __forceinline__ void fragment_epilogue(const GemmArgs &g, int64_t row0, int64_t col, float (&v)[16]) {
  float e[16];
  if (g.resid) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t row = row0 + 8 * (r >> 2) + (r & 3);
      e[r] = (!GUARD || (row < g.M && col < g.N)) ? g.resid[row * g.ldr + col] : 0.f;
    }
  }
  const float b = (g.bias && (!GUARD || col < g.N)) ? g.bias[col] : 0.f;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    float x = v[r];
    if (g.bias) x = __fadd_rn(x, b);
    if (g.resid) x = __fadd_rn(e[r], x);
    v[r] = x;
  }
}

// Map a linear workgroup id to an output tile (tm, tn), grouping the tiles
// each XCD receives.  Workgroup w runs on XCD w % 8.
__device__ __forceinline__ void tile_of(int w, int tiles_m, int tiles_n, int *tm, int *tn) {
  const int total = tiles_m * tiles_n;
  int t = w;
  if ((total & 7) == 0) t = (w & 7) * (total >> 3) + (w >> 3);
  // Within the XCD-ordered sequence, walk groups of GROUP_M tile rows.
  constexpr int GROUP_M = 4;
  const int group_size = GROUP_M * tiles_n;
  const int g = t / group_size;
  const int first_m = g * GROUP_M;
  const int gm = (tiles_m - first_m) < GROUP_M ? (tiles_m - first_m) : GROUP_M;
  const int in_g = t - g * group_size;
  *tm = first_m + in_g % gm;
  *tn = in_g / gm;
}

template <typename T, typename SA, typename SB, typename TO, int BM, int BN, int WM, int WN, bool AK, bool BKC,
          bool GUARD, int STORE_AT = 3>
__global__ void __launch_bounds__(WM *WN * 64) gemm_kernel(GemmArgs g) {
  constexpr int NT = WM * WN * 64;
  constexpr int BK = 128 / sizeof(T);
  constexpr int WTM = BM / WM, WTN = BN / WN;  // wave tile
  constexpr int TM = WTM / 32, TN = WTN / 32;  // 32x32 MFMA tiles per wave
  static_assert(TM >= 1 && TN >= 1, "wave tile");
  constexpr int A_BYTES = BM * 128, B_BYTES = BN * 128;
  constexpr int STAGE = A_BYTES + B_BYTES;
  extern __shared__ __attribute__((aligned(16))) char smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  int tm, tn;
  tile_of(blockIdx.x, g.tiles_m, g.tiles_n, &tm, &tn);
  const int64_t m0 = static_cast<int64_t>(tm) * BM, n0 = static_cast<int64_t>(tn) * BN;
  const int64_t z = blockIdx.y;
  const int64_t zo = z / g.per_group, zi = z - zo * g.per_group;
  const SA *A = static_cast<const SA *>(g.a) + zo * g.sa2 + zi * g.sa;
  const SB *B = static_cast<const SB *>(g.b) + zo * g.sb2 + zi * g.sb;
  TO *C = static_cast<TO *>(g.c) + zo * g.sc2 + zi * g.sc;
  int64_t Kz = g.K;
  if (g.kc > 0) {
    // Split-K slice blockIdx.z: k in [ks, ks + Kz), its partial product
    // written to slice z of an [S, M, N] buffer.
    const int64_t ks = static_cast<int64_t>(blockIdx.z) * g.kc;
    Kz = g.K - ks < g.kc ? g.K - ks : g.kc;
    A += AK ? ks : ks * g.lda;
    B += BKC ? ks : ks * g.ldb;
    C += static_cast<int64_t>(blockIdx.z) * g.M * g.ldc;
  }

  TileLoader<T, SA, BM, NT, AK, GUARD> la;
  TileLoader<T, SB, BN, NT, BKC, GUARD> lb;

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int64_t ktiles = (Kz + BK - 1) / BK;
  la.load(A, g.lda, m0, 0, g.M, Kz, tid);
  lb.load(B, g.ldb, n0, 0, g.N, Kz, tid);
  la.store(smem, tid);
  lb.store(smem + A_BYTES, tid);
  __syncthreads();

  const int lrow = lane & 31, lhalf = lane >> 5;
  // Fragment registers, double-buffered over the four chunk pairs of a
  // k-tile: the reads for pair p + 1 are issued before the MFMAs of pair p.
  Chunk fa[2][TM], fb[2][TN];
  auto read_frags = [&](const char *a_s, const char *b_s, int p, int buf) {
    const int c = 2 * p + lhalf;
#pragma unroll
    for (int i = 0; i < TM; ++i) fa[buf][i].u = *reinterpret_cast<const uint4 *>(a_s + lds_off(wm * WTM + i * 32 + lrow, c));
#pragma unroll
    for (int j = 0; j < TN; ++j) fb[buf][j].u = *reinterpret_cast<const uint4 *>(b_s + lds_off(wn * WTN + j * 32 + lrow, c));
  };
  auto mfmas = [&](int buf) {
    if constexpr (sizeof(T) == 2) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, fa[buf][i].u),
                                                              __builtin_bit_cast(bf16x8, fb[buf][j].u), acc[i][j], 0, 0, 0);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[buf][i].f[e], fb[buf][j].f[e], acc[i][j], 0, 0, 0);
    }
  };

  read_frags(smem, smem + A_BYTES, 0, 0);
  for (int64_t kt = 0; kt < ktiles; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < ktiles;
    if (more) {
      la.load(A, g.lda, m0, (kt + 1) * BK, g.M, Kz, tid);
      lb.load(B, g.ldb, n0, (kt + 1) * BK, g.N, Kz, tid);
    }
    const char *a_s = smem + cur * STAGE;
    const char *b_s = a_s + A_BYTES;
    char *nxt = smem + (cur ^ 1) * STAGE;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      if (p < 3) read_frags(a_s, b_s, p + 1, (p + 1) & 1);
      mfmas(p & 1);
      // The other stage was last read before the previous barrier: the next
      // tile may be written into it while this one is still being consumed.
      if (p == STORE_AT && more) {
        la.store(nxt, tid);
        lb.store(nxt + A_BYTES, tid);
      }
    }
    __syncthreads();
    if (more) read_frags(nxt, nxt + A_BYTES, 0, 0);
  }

  // Epilogue: lane holds column (lane & 31) and rows 8*(r/4) + 4*(lane/32) + r%4.
  const bool epi = g.bias != nullptr || g.resid != nullptr;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int64_t col = n0 + wn * WTN + j * 32 + lrow;
      const int64_t rb = m0 + wm * WTM + i * 32 + 4 * lhalf;
      float v[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) v[r] = acc[i][j][r];
      if (epi) fragment_epilogue<GUARD>(g, rb, col, v);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = rb + 8 * (r >> 2) + (r & 3);
        if (!GUARD || (row < g.M && col < g.N)) {
          if constexpr (sizeof(TO) == 2) C[row * g.ldc + col] = f32_to_bf16_bits(v[r]);
          else C[row * g.ldc + col] = v[r];
        }
      }
    }
  }
}

// ------------------------------------- F32 operands on the BF16 matrix cores
// The fast matmul mode for F32 operands.  Each F32 element a is split as
// a = hi + lo + e with hi = bf16(a) and lo = bf16(a - hi) (a - hi is exact,
// |e| <= 2^-18 |a|), and a product a b is taken as hi_a hi_b + hi_a lo_b +
// lo_a hi_b on v_mfma_f32_32x32x16_bf16, accumulated in F32; a BF16 operand
// has no lo part (two products, error <= 2^-18 |a||b|).  Per product the error
// is at most 3 * 2^-18 |a||b| -- far inside the reference's own fast mode
// (TF32 operands, crates/burn-tt/src/matmul_mode.rs:1-8) -- and the matrix
// cores run 16x the F32 rate, so 3 (2) products cost 5.3x (8x) less than
// v_mfma_f32_32x32x2f32.  The split happens in registers between the global
// load and the LDS write: no pass over HBM, no extra launch.

// Tile loader of the split kernel: ROWS rows x 64 k of an F32 (split into hi
// and lo planes) or BF16 (hi plane only) operand, into swizzled 128-byte LDS
// rows.  KCONTIG: source element (r, k) at src[r * ld + k], a unit is 8
// consecutive k of one row; otherwise at src[k * ld + r], a unit is an 8 x 8
// block (8 k x 8 rows) transposed in registers.  A thread whose index runs
// past the last unit idles.
template <typename S, int ROWS, int NT, bool KCONTIG, bool GUARD>
struct SplitLoader {
  static constexpr bool SPLIT = sizeof(S) == 4;
  static constexpr int UNITS = KCONTIG ? ROWS * 8 : (ROWS / 8) * 8;
  static constexpr int NU = (UNITS + NT - 1) / NT;
  static constexpr bool EVEN = UNITS % NT == 0;
  static constexpr int RAW = KCONTIG ? 8 : 64;
  static_assert(ROWS % 8 == 0, "tile rows a multiple of 8");
  S raw[NU][RAW];

  __device__ __forceinline__ void load(const S *src, int64_t ld, int64_t r0, int64_t k0, int64_t rows_total,
                                       int64_t k_total, int tid) {
#pragma unroll
    for (int i = 0; i < NU; ++i) {
      const int q = tid + i * NT;
      if (!EVEN && q >= UNITS) break;
      if constexpr (KCONTIG) {
        const int r = q / 8, c = q % 8;
        const int64_t gr = r0 + r, gk = k0 + c * 8;
        const S *p = src + gr * ld + gk;
        int valid = 8;
        if constexpr (GUARD) {
          valid = (gr < rows_total) ? static_cast<int>(k_total - gk) : 0;
          valid = valid < 0 ? 0 : (valid > 8 ? 8 : valid);
        }
        fetch(p, valid, raw[i], 0);
      } else {
        const int kb = q % 8, rb = q / 8;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int64_t gk = k0 + kb * 8 + e, gr = r0 + rb * 8;
          const S *p = src + gk * ld + gr;
          int valid = 8;
          if constexpr (GUARD) {
            valid = (gk < k_total) ? static_cast<int>(rows_total - gr) : 0;
            valid = valid < 0 ? 0 : (valid > 8 ? 8 : valid);
          }
          fetch(p, valid, raw[i], 8 * e);
        }
      }
    }
  }

  // Eight elements at p into raw[o .. o + 7]: vector loads when all are in
  // range and aligned, else element by element (zero past `valid`).
  __device__ __forceinline__ static void fetch(const S *p, int valid, S *dst, int o) {
    if (valid == 8 && (!GUARD || (reinterpret_cast<uintptr_t>(p) & 15) == 0)) {
      if constexpr (sizeof(S) == 4) {
        const float4 a = *reinterpret_cast<const float4 *>(p);
        const float4 b = *reinterpret_cast<const float4 *>(p + 4);
        dst[o + 0] = a.x; dst[o + 1] = a.y; dst[o + 2] = a.z; dst[o + 3] = a.w;
        dst[o + 4] = b.x; dst[o + 5] = b.y; dst[o + 6] = b.z; dst[o + 7] = b.w;
      } else {
        Chunk c;
        c.u = *reinterpret_cast<const uint4 *>(p);
#pragma unroll
        for (int e = 0; e < 8; ++e) dst[o + e] = c.h[e];
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) dst[o + e] = e < valid ? p[e] : S(0);
    }
  }

  // One chunk (8 k of one row) into the hi plane, and its remainders into the
  // lo plane for an F32 source (split_bf16x2: two values an instruction).
  __device__ __forceinline__ static void put(char *hi_plane, char *lo_plane, int r, int c, const S (&v)[8]) {
    Chunk h, l;
    if constexpr (SPLIT) {
      uint32_t hw[4], lw[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) split_bf16x2(v[2 * e], v[2 * e + 1], hw[e], lw[e]);
      h.u = make_uint4(hw[0], hw[1], hw[2], hw[3]);
      l.u = make_uint4(lw[0], lw[1], lw[2], lw[3]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) h.h[e] = v[e];
    }
    *reinterpret_cast<uint4 *>(hi_plane + lds_off(r, c)) = h.u;
    if constexpr (SPLIT) *reinterpret_cast<uint4 *>(lo_plane + lds_off(r, c)) = l.u;
  }

  __device__ __forceinline__ void store(char *hi_plane, char *lo_plane, int tid) const {
#pragma unroll
    for (int i = 0; i < NU; ++i) {
      const int q = tid + i * NT;
      if (!EVEN && q >= UNITS) break;
      if constexpr (KCONTIG) {
        S v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = raw[i][e];
        put(hi_plane, lo_plane, q / 8, q % 8, v);
      } else {
        const int kb = q % 8, rb = q / 8;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          S v[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = raw[i][8 * e + j];  // k = e of row rb * 8 + j
          put(hi_plane, lo_plane, rb * 8 + j, kb, v);
        }
      }
    }
  }
};

template <typename SA, typename SB, typename TO, int BM, int BN, int WM, int WN, bool AK, bool BKC, bool GUARD>
__global__ void __launch_bounds__(WM *WN * 64) gemm_split_kernel(GemmArgs g) {
  constexpr int NT = WM * WN * 64;
  constexpr int BK = 64;
  constexpr bool LA = sizeof(SA) == 4, LB = sizeof(SB) == 4;  // operands with a lo plane
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  static_assert(TM >= 1 && TN >= 1, "wave tile");
  constexpr int A_PLANE = BM * 128, B_PLANE = BN * 128;
  constexpr int A_BYTES = A_PLANE * (LA ? 2 : 1), B_BYTES = B_PLANE * (LB ? 2 : 1);
  constexpr int STAGE = A_BYTES + B_BYTES;
  extern __shared__ __attribute__((aligned(16))) char smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  int tm, tn;
  tile_of(blockIdx.x, g.tiles_m, g.tiles_n, &tm, &tn);
  const int64_t m0 = static_cast<int64_t>(tm) * BM, n0 = static_cast<int64_t>(tn) * BN;
  const int64_t z = blockIdx.y;
  const int64_t zo = z / g.per_group, zi = z - zo * g.per_group;
  const SA *A = static_cast<const SA *>(g.a) + zo * g.sa2 + zi * g.sa;
  const SB *B = static_cast<const SB *>(g.b) + zo * g.sb2 + zi * g.sb;
  TO *C = static_cast<TO *>(g.c) + zo * g.sc2 + zi * g.sc;
  int64_t Kz = g.K;
  if (g.kc > 0) {
    const int64_t ks = static_cast<int64_t>(blockIdx.z) * g.kc;
    Kz = g.K - ks < g.kc ? g.K - ks : g.kc;
    A += AK ? ks : ks * g.lda;
    B += BKC ? ks : ks * g.ldb;
    C += static_cast<int64_t>(blockIdx.z) * g.M * g.ldc;
  }

  SplitLoader<SA, BM, NT, AK, GUARD> la;
  SplitLoader<SB, BN, NT, BKC, GUARD> lb;

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int64_t ktiles = (Kz + BK - 1) / BK;
  la.load(A, g.lda, m0, 0, g.M, Kz, tid);
  lb.load(B, g.ldb, n0, 0, g.N, Kz, tid);
  la.store(smem, smem + A_PLANE, tid);
  lb.store(smem + A_BYTES, smem + A_BYTES + B_PLANE, tid);
  __syncthreads();

  const int lrow = lane & 31, lhalf = lane >> 5;
  for (int64_t kt = 0; kt < ktiles; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < ktiles;
    if (more) {
      la.load(A, g.lda, m0, (kt + 1) * BK, g.M, Kz, tid);
      lb.load(B, g.ldb, n0, (kt + 1) * BK, g.N, Kz, tid);
    }
    const char *a_s = smem + cur * STAGE;
    const char *b_s = a_s + A_BYTES;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int c = 2 * p + lhalf;
      Chunk ah[TM], al[TM], bh[TN], bl[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int off = lds_off(wm * WTM + i * 32 + lrow, c);
        ah[i].u = *reinterpret_cast<const uint4 *>(a_s + off);
        if constexpr (LA) al[i].u = *reinterpret_cast<const uint4 *>(a_s + A_PLANE + off);
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int off = lds_off(wn * WTN + j * 32 + lrow, c);
        bh[j].u = *reinterpret_cast<const uint4 *>(b_s + off);
        if constexpr (LB) bl[j].u = *reinterpret_cast<const uint4 *>(b_s + B_PLANE + off);
      }
      // The small cross terms first, then the head product.
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          if constexpr (LA)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, al[i].u),
                                                                __builtin_bit_cast(bf16x8, bh[j].u), acc[i][j], 0, 0, 0);
          if constexpr (LB)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, ah[i].u),
                                                                __builtin_bit_cast(bf16x8, bl[j].u), acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, ah[i].u),
                                                              __builtin_bit_cast(bf16x8, bh[j].u), acc[i][j], 0, 0, 0);
        }
    }
    if (more) {
      // The other stage was last read before the previous barrier.
      char *nxt = smem + (cur ^ 1) * STAGE;
      la.store(nxt, nxt + A_PLANE, tid);
      lb.store(nxt + A_BYTES, nxt + A_BYTES + B_PLANE, tid);
    }
    __syncthreads();
  }

  // Epilogue: lane holds column (lane & 31) and rows 8*(r/4) + 4*(lane/32) + r%4.
  const bool epi = g.bias != nullptr || g.resid != nullptr;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int64_t col = n0 + wn * WTN + j * 32 + lrow;
      const int64_t rb = m0 + wm * WTM + i * 32 + 4 * lhalf;
      float v[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) v[r] = acc[i][j][r];
      if (epi) fragment_epilogue<GUARD>(g, rb, col, v);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = rb + 8 * (r >> 2) + (r & 3);
        if (!GUARD || (row < g.M && col < g.N)) {
          if constexpr (sizeof(TO) == 2) C[row * g.ldc + col] = f32_to_bf16_bits(v[r]);
          else C[row * g.ldc + col] = v[r];
        }
      }
    }
  }
}

// ------------------------------------------- BF16: HBM -> LDS direct path
// The BF16 kernel for exactly tiled shapes.  Operand tiles move from HBM to
// LDS with `global_load_lds_dwordx4` (each lane's 16 bytes land at
// base + 16 * lane), so no staging registers and no LDS store instructions
// are spent on them, and the next k-tile streams in while the current one is
// multiplied.  An operand whose k is contiguous keeps the swizzled 128-byte
// rows above; one whose m/n is contiguous is stored as it lies, [k][rows], and
// its MFMA fragments are read with `ds_read_b64_tr_b16`, which hands lane j of
// each 16-lane group element j % 4 of the 8 bytes that lane 4 t + j / 4 of the
// group addressed (t = 0..3): lane i addressing row k0 + i / 4, columns
// n0 + 4 (i % 4) .. + 3 gives lane j the four k of column n0 + j.  Chunk c of
// row k of such a tile is stored at chunk c ^ (4 (k % 4)), so the 16 rows x 64
// bytes a transposed fragment read touches cover all 64 banks.
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;

template <int ROWS, bool KCONTIG, int BK>
struct DmaOperand {
  static constexpr int BYTES = ROWS * BK * 2;  // tile bytes (ROWS x BK BF16)
  static constexpr int BLOCKS = BYTES / 1024;
  static constexpr int READS = KCONTIG ? 1 : 2;  // LDS reads per fragment
  // k-contiguous tiles: RB-byte rows of CPR 16-byte chunks, chunk c of row r
  // stored at c ^ swz(r) -- for 128-byte rows r & 7, for 64-byte rows
  // (r / 4) & 3 -- so 32 rows at one logical chunk spread over all banks.
  static constexpr int RB = KCONTIG ? 2 * BK : 2 * ROWS;
  static constexpr int CPR = RB / 16;
  static constexpr int RPB = 1024 / RB;  // rows per 1 KiB block
  static_assert(BK == 32 || BK == 64, "k tile");
  static_assert(KCONTIG || ROWS >= 128, "transposed-read swizzle needs rows of 16+ chunks");
  __device__ __forceinline__ static int swz(int r) {
    if constexpr (BK == 64) return r & 7;
    else return (r >> 2) & 3;
  }

  // A wave moves its share of a tile's 1 KiB blocks.  Each address is a
  // wave-uniform block base (SGPRs) plus one 32-bit per-lane byte offset.
  // The instruction is written out (with M0, its LDS base, set just before)
  // rather than left to the compiler, which would otherwise wait for every
  // DMA still in flight before any later LDS read; the kernel counts its own
  // DMA instead (wait_vmcnt before each barrier, and 0 before it ends).
  // Where this wave's share of a tile comes from: a per-lane byte offset and
  // the wave's first block base (block i at base + i * ustep).
  struct Src {
    uint32_t voff;
    const char *base;
    int64_t ustep;
    // Rows past `limit` (an edge tile of a k-contiguous operand whose row
    // count is not a multiple of the tile, and a multiple of RPB): such a
    // block is read from `clamp` (the last whole block of rows) instead, so
    // no read leaves the operand; those rows only feed results that are not
    // stored.  limit = 0: no edge.
    int64_t first_row, limit;
    const char *clamp;
  };
  // A wave's DMA instructions per tile: its blocks wave, wave + NW, ...;
  // where NW does not divide the blocks, a wave with one fewer repeats its
  // last (the same bytes into the same LDS block), so every wave issues the
  // same count and the counted waits stay exact.
  template <int NW>
  static constexpr int per_wave() {
    return (BLOCKS + NW - 1) / NW;
  }
  template <int NW>
  __device__ __forceinline__ static Src src_of(const uint16_t *src, int64_t ld, int64_t r0, int64_t k0, int wave,
                                               int lane) {
    static_assert(BLOCKS >= NW, "blocks per wave");
    const int lr = (lane * 16) / RB;          // row of this lane within its block
    const int pch = ((lane * 16) % RB) >> 4;  // physical chunk it fills
    uint32_t voff;
    int64_t base_off, ustep;  // bytes
    if constexpr (KCONTIG) {
      // Block b covers rows RPB b .. RPB b + RPB - 1 (RPB a multiple of 8 or
      // 16), so swz(row) = swz(lr).
      const int c = pch ^ swz(lr);
      voff = static_cast<uint32_t>((lr * ld + c * 8) * 2);
      base_off = ((r0 + RPB * wave) * ld + k0) * 2;
    } else {
      // k row of this lane: RPB b + lr; RPB * NW is a multiple of 4, so
      // k % 4 = (RPB wave + lr) % 4 for every block this wave loads.
      const int kq = (RPB * wave + lr) & 3;
      const int c = pch ^ (4 * kq);
      voff = static_cast<uint32_t>((lr * ld + c * 8) * 2);
      base_off = ((k0 + RPB * wave) * ld + r0) * 2;
    }
    ustep = static_cast<int64_t>(RPB) * NW * ld * 2;
    return Src{voff, reinterpret_cast<const char *>(src) + base_off, ustep, 0, 0, nullptr};
  }
  // src_of for a k-contiguous operand of `rows` rows (a multiple of RPB) whose
  // last tile runs past them.
  template <int NW>
  __device__ __forceinline__ static Src src_edge(const uint16_t *src, int64_t ld, int64_t r0, int64_t k0, int wave,
                                                 int lane, int64_t rows) {
    Src sr = src_of<NW>(src, ld, r0, k0, wave, lane);
    if constexpr (!KCONTIG) return sr;  // only k-contiguous operands take an edge
    sr.first_row = r0 + RPB * wave;
    sr.limit = rows;
    sr.clamp = reinterpret_cast<const char *>(src) + ((rows - RPB) * ld + k0) * 2;
    return sr;
  }

  // The DMA instruction of this wave's block i of the tile into `lds`.
  template <int NW>
  __device__ __forceinline__ static void issue(const Src &sr, int i, char *lds, int wave) {
    if constexpr (BLOCKS % NW != 0) {
      if (i * NW + wave >= BLOCKS) i -= 1;  // this wave's repeat of its last block
    }
    const int b = i * NW + wave;
    const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void *)(lds)));
    const uint32_t m0v = __builtin_amdgcn_readfirstlane(lds0 + b * 1024);
    const char *p = sr.base + i * sr.ustep;
    if (sr.limit && sr.first_row + static_cast<int64_t>(i) * RPB * NW >= sr.limit) p = sr.clamp;
    const char *gb = reinterpret_cast<const char *>(
        static_cast<uint64_t>(static_cast<uint32_t>(
            __builtin_amdgcn_readfirstlane(static_cast<int>(reinterpret_cast<uintptr_t>(p))))) |
        (static_cast<uint64_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(reinterpret_cast<uintptr_t>(p) >> 32)))
         << 32));
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
                 :
                 : "s"(m0v), "v"(sr.voff), "s"(gb)
                 : "memory", "m0");
#pragma clang diagnostic pop
  }

  // Issue this wave's share of the tile's 1 KiB blocks (all of them).
  template <int NW>
  __device__ __forceinline__ static void load(const uint16_t *src, int64_t ld, int64_t r0, int64_t k0, char *lds,
                                              int wave, int lane, int64_t rows = 0) {
    const Src sr = rows ? src_edge<NW>(src, ld, r0, k0, wave, lane, rows) : src_of<NW>(src, ld, r0, k0, wave, lane);
#pragma unroll
    for (int i = 0; i < per_wave<NW>(); ++i) issue<NW>(sr, i, lds, wave);
  }

  // The 8 BF16 of lane `lane` for the 32-row fragment at `row0`, k step p.
  __device__ __forceinline__ static uint4 frag(const char *lds, int row0, int p, int lane) {
    if constexpr (KCONTIG) {
      const int r = row0 + (lane & 31);
      const int c = 2 * p + (lane >> 5);
      return *reinterpret_cast<const uint4 *>(lds + r * RB + ((c ^ swz(r)) << 4));
    } else {
      const int i = lane & 15;
      const int nhalf = (lane >> 4) & 1, kg = lane >> 5;
      const int n = row0 + 16 * nhalf + 4 * (i & 3);
      const int kbase = p * 16 + kg * 8 + (i >> 2);
      uint4 out;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int k = kbase + 4 * h;
        const int pch = (n >> 3) ^ (4 * (k & 3));
        const char *addr = lds + k * RB + pch * 16 + ((n & 7) >> 2) * 8;
        v4i16 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16 *)(addr));
        if (h == 0) { out.x = __builtin_bit_cast(uint2, v).x; out.y = __builtin_bit_cast(uint2, v).y; }
        else { out.z = __builtin_bit_cast(uint2, v).x; out.w = __builtin_bit_cast(uint2, v).y; }
      }
      return out;
    }
  }
};

// `s_waitcnt vmcnt(N)`, the other counters left alone.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// The static LDS stage S of NS (unused stages collapse to 16 bytes).
#define MI_DMA_STAGES(STAGE, NS)                                                            \
  __shared__ __attribute__((aligned(1024))) char st0[STAGE];                                 \
  __shared__ __attribute__((aligned(1024))) char st1[STAGE];                                 \
  __shared__ __attribute__((aligned(1024))) char st2[(NS) > 2 ? (STAGE) : 16];               \
  __shared__ __attribute__((aligned(1024))) char st3[(NS) > 3 ? (STAGE) : 16];               \
  __shared__ __attribute__((aligned(1024))) char st4[(NS) > 4 ? (STAGE) : 16];               \
  char *const stages[5] = {st0, st1, st2, st3, st4};

// ------------------------------------- BF16: pipelined direct path
// The direct path with the waits taken off the MFMA stream.  k-tiles of 32
// (two MFMA k steps) in NS >= 3 LDS stages; every step's fragments are read
// one step ahead into the other of two register buffers, across tile
// boundaries too, so an MFMA never waits on an LDS read issued just before
// it.  The one barrier per tile sits before the tile's last step: by then
// every wave has finished the previous tile (so its stage can be refilled)
// and this thread's DMA of the next tile has landed (so, after the barrier,
// every wave's has), which lets the last step's MFMAs cover the first reads
// of the next tile.  Scheduling fences keep the compiler from sinking the
// reads back down to their uses.
template <typename OA, typename OB, int TM, int TN, int WTM, int WTN>
__device__ __forceinline__ void pipe_reads(uint4 (&fa)[TM], uint4 (&fb)[TN], const char *stage, int p, int wm, int wn,
                                           int lane) {
#pragma unroll
  for (int i = 0; i < TM; ++i) fa[i] = OA::frag(stage, wm * WTM + i * 32, p, lane);
#pragma unroll
  for (int j = 0; j < TN; ++j) fb[j] = OB::frag(stage + OA::BYTES, wn * WTN + j * 32, p, lane);
}

// Scheduling directive for one step: the MFMAs in order, the first ones
// each followed by PER of the NR LDS reads of the next step, so every read
// is issued early in the step (and lands before the next one) while no more
// reads are in flight at the step's first MFMA than its own operands.
template <int Q, int MF, int NR, int PER>
__device__ __forceinline__ void mfma_then_reads() {
  if constexpr (Q < MF) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
    if constexpr (Q * PER < NR)
      __builtin_amdgcn_sched_group_barrier(0x100, (NR - Q * PER) < PER ? (NR - Q * PER) : PER, 0);  // LDS reads
    mfma_then_reads<Q + 1, MF, NR, PER>();
  }
}

template <int TM, int TN>
__device__ __forceinline__ void pipe_mfma(f32x16 (&acc)[TM][TN], const uint4 (&fa)[TM], const uint4 (&fb)[TN]) {
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, fa[i]),
                                                          __builtin_bit_cast(bf16x8, fb[j]), acc[i][j], 0, 0, 0);
}

// The rotary tables' rows of a block's BM result rows (cos, then sin), read
// into the LDS stages once the main loop is done with them: row lr of a table
// at stage (table (BM / RPS) + lr / RPS), RPS rows of 64 floats a stage.  One
// request a thread per 16 bytes, all in flight together, instead of each
// wavefront's 64 scalar loads a fragment.
// Row lr of rotary table tbl (0 cos, 1 sin) among the stages (a select
// between stages named at compile time, not an index into a pointer array,
// which would live in scratch memory).
template <int BM, int RPS>
__device__ __forceinline__ char *qkv_table_row(char *const (&stages)[5], int tbl, int lr) {
  static_assert(BM / RPS == 1 || BM / RPS == 2, "a table in one or two stages");
  char *s0 = tbl ? stages[BM / RPS] : stages[0];
  if constexpr (BM / RPS == 2) {
    char *s1 = tbl ? stages[BM / RPS + 1] : stages[1];
    s0 = lr < RPS ? s0 : s1;
  }
  return s0 + (lr % RPS) * 256;
}

template <int BM, int NS, int STAGE, int NT>
__device__ __forceinline__ void qkv_tables(const QkvTail &t, int64_t m0, char *const (&stages)[5], int tid) {
  constexpr int RPS = STAGE / 256;
  static_assert(RPS >= 1 && 2 * BM <= NS * RPS, "rotary tables in the stages");
  constexpr int PER = 2 * BM * 16 / NT, BATCH = PER < 8 ? PER : 8;  // 16-byte pieces a thread, in batches
  static_assert(PER * NT == 2 * BM * 16 && PER % BATCH == 0, "table pieces a thread");
  // The block's rows in one sequence (consecutive positions): no division a row.
  const int64_t b0 = m0 / t.seq, p0 = m0 - b0 * t.seq;
  const bool one = p0 + BM <= t.seq;
  auto src = [&](int c) {
    const int tbl = c / (BM * 16), rem = c - tbl * (BM * 16), lr = rem >> 4, q4 = rem & 15;
    int64_t pos;
    if (one) {
      pos = t.pos0 + p0 + lr;
    } else {
      const int64_t row = m0 + lr, b = row / t.seq;
      pos = t.pos0 + (row - b * t.seq);
    }
    return reinterpret_cast<const float4 *>((tbl ? t.sin : t.cos) + pos * 64 + 4 * q4);
  };
  auto dst = [&](int c) {
    const int tbl = c / (BM * 16), rem = c - tbl * (BM * 16), lr = rem >> 4, q4 = rem & 15;
    return reinterpret_cast<float4 *>(qkv_table_row<BM, RPS>(stages, tbl, lr) + 16 * q4);
  };
#pragma unroll
  for (int u0 = 0; u0 < PER; u0 += BATCH) {
    float4 v[BATCH];
#pragma unroll
    for (int u = 0; u < BATCH; ++u) v[u] = *src(tid + (u0 + u) * NT);
#pragma unroll
    for (int u = 0; u < BATCH; ++u) *dst(tid + (u0 + u) * NT) = v[u];
  }
}

// The q|k|v tail of a wavefront whose 64 columns are head hb / 64: fragment
// 0 holds its columns j = lane % 32, fragment 1 columns j + 32 -- each
// other's RoPE partners -- at rows row0 + 32 i + 8 (r / 4) + r % 4, the
// block's rows from m0.  The rotary entries come from the LDS copy
// qkv_tables made (RPS rows a stage).
template <int TM, int BM, int RPS>
__device__ __forceinline__ void qkv_tail(const GemmArgs &g, const f32x16 (&acc)[TM][2], int64_t row0, int64_t hb,
                                         int j, int64_t m0, char *const (&stages)[5]) {
  const QkvTail &t = g.qkv;
  if (hb >= g.N) return;  // an edge tile's columns past the last head
  const int h = static_cast<int>(hb >> 6);
  const bool rope = h < t.heads + t.kvh;
  // The wavefront's head: a query head (its kv group and place in it), or
  // kv head jj's key or value.
  const int G = t.heads / t.kvh;
  const bool isq = h < t.heads, isk = !isq && rope;
  const int kvq = isq ? h / G : 0, gq = isq ? h - kvq * G : 0;
  const int jj = isq ? 0 : (isk ? h - t.heads : h - t.heads - t.kvh);
  // A fragment's 32 rows (32-aligned) lie in one sequence when seq is a
  // multiple of 32: one division a fragment, not two a value.
  const bool whole = (t.seq & 31) == 0;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int64_t fb = (row0 + i * 32) & ~static_cast<int64_t>(31);
    const int64_t fbs = whole ? fb / t.seq : 0, fps = fb - fbs * t.seq;
    auto seq_of = [&](int64_t row, int64_t &b, int64_t &p) {
      if (whole) {
        b = fbs;
        p = fps + (row - fb);
      } else {
        b = row / t.seq;
        p = row - b * t.seq;
      }
    };
    float c0[16], c1[16], s0[16], s1[16];
    if (rope) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int lr = static_cast<int>(row0 + i * 32 + 8 * (r >> 2) + (r & 3) - m0);
        const float *cr = reinterpret_cast<const float *>(qkv_table_row<BM, RPS>(stages, 0, lr));
        const float *sr = reinterpret_cast<const float *>(qkv_table_row<BM, RPS>(stages, 1, lr));
        c0[r] = cr[j];
        c1[r] = cr[j + 32];
        s0[r] = sr[j];
        s1[r] = sr[j + 32];
      }
    }
    if (whole) {
      // The fragment's rows in one sequence: the wavefront's destination rows
      // are base + p * stride for its head (q rows natural or grouped, or the
      // k or v cache rows), so each value's address is a constant step from
      // one base a fragment -- not qkv_put's divisions and products per value.
      const int64_t b = fbs, p0 = fps + (row0 + i * 32 - fb);  // the position of value r = 0
      int64_t base, stride;
      if (isq) {
        base = t.grouped ? ((b * t.kvh + kvq) * t.seq + p0) * G + gq : (b * t.seq + p0) * t.heads + h;
        stride = t.grouped ? G : t.heads;
      } else {
        base = (b * t.kvh + jj) * t.maxc + t.pos0 + p0;
        stride = 1;
      }
      float *qd = t.q + base * 64 + j;
      float *cf = static_cast<float *>(isk ? t.kc : t.vc) + base * 64 + j;
      uint16_t *ch = static_cast<uint16_t *>(isk ? t.kc : t.vc) + base * 64 + j;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t o = (8 * (r >> 2) + (r & 3)) * stride * 64;
        float y0 = acc[i][0][r], y1 = acc[i][1][r];
        if (rope) rope_pair(acc[i][0][r], acc[i][1][r], c0[r], c1[r], s0[r], s1[r], y0, y1);
        if (isq) {
          qd[o] = y0;
          qd[o + 32] = y1;
        } else if (t.mode == QKV_BF16) {
          ch[o] = f32_to_bf16_bits(y0);
          ch[o + 32] = f32_to_bf16_bits(y1);
        } else {
          cf[o] = y0;
          cf[o + 32] = y1;
        }
      }
      continue;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t row = row0 + i * 32 + 8 * (r >> 2) + (r & 3);
      int64_t b, p;
      seq_of(row, b, p);
      float y0 = acc[i][0][r], y1 = acc[i][1][r];
      if (rope) rope_pair(acc[i][0][r], acc[i][1][r], c0[r], c1[r], s0[r], s1[r], y0, y1);
      qkv_put(t, row, b, p, h, j, y0, y1);
    }
  }
}

template <typename TO, int BM, int BN, int NS, bool AK, bool BKC, int WM, int WN, bool GN>
__device__ __forceinline__ void gemm_pipe_body(const GemmArgs &g) {
  constexpr int BK = 32;  // two MFMA k steps per tile
  constexpr int NW = WM * WN;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  using OA = DmaOperand<BM, AK, BK>;
  using OB = DmaOperand<BN, BKC, BK>;
  constexpr int STAGE = OA::BYTES + OB::BYTES;
  constexpr int PA = OA::template per_wave<NW>(), PB = OB::template per_wave<NW>();
  constexpr int PER_TILE = PA + PB;  // this thread's DMA instructions per tile
  static_assert(NS >= 3 && NS <= 5, "stages");
  static_assert(NS * STAGE <= 160 * 1024, "LDS");
  constexpr int MF = TM * TN;                          // MFMAs per step
  constexpr int NR = TM * OA::READS + TN * OB::READS;  // LDS reads per step
  MI_DMA_STAGES(STAGE, NS)

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  int tm, tn;
  tile_of(blockIdx.x, g.tiles_m, g.tiles_n, &tm, &tn);
  const int64_t m0 = static_cast<int64_t>(tm) * BM, n0 = static_cast<int64_t>(tn) * BN;
  const int64_t z = blockIdx.y;
  const int64_t zo = z / g.per_group, zi = z - zo * g.per_group;
  const uint16_t *A = static_cast<const uint16_t *>(g.a) + zo * g.sa2 + zi * g.sa;
  const uint16_t *B = static_cast<const uint16_t *>(g.b) + zo * g.sb2 + zi * g.sb;
  TO *C = static_cast<TO *>(g.c) + zo * g.sc2 + zi * g.sc;

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int64_t ktiles = g.K / BK;
  // Tiles past the last reload the last into a stage nobody reads again, so
  // every thread issues PER_TILE DMA instructions per tile and the counted
  // waits stay exact.
  auto kclamp = [&](int64_t t) { return (t < ktiles ? t : ktiles - 1) * BK; };
  // B's k of tile t: wrapped modulo its own extent when A repeats it.
  auto kbof = [&](int64_t t) { return g.kb ? kclamp(t) % g.kb : kclamp(t); };
  // GN: the last column tile runs past N (B k-contiguous, N a multiple of
  // its block rows): those B rows are read from the last whole block, their
  // results not stored.
  const int64_t brows = GN ? g.N : 0;
#pragma unroll
  for (int s = 0; s < NS - 1; ++s) {
    OA::template load<NW>(A, g.lda, m0, kclamp(s), stages[s], wave, lane);
    OB::template load<NW>(B, g.ldb, n0, kbof(s), stages[s] + OA::BYTES, wave, lane, brows);
  }
  // Tile 0 landed everywhere (tiles 1 .. NS-2 may be in flight).
  wait_vmcnt<(NS - 2) * PER_TILE>();
  __builtin_amdgcn_s_barrier();
  uint4 fa0[TM], fb0[TN], fa1[TM], fb1[TN];
  pipe_reads<OA, OB, TM, TN, WTM, WTN>(fa0, fb0, stages[0], 0, wm, wn, lane);
  for (int64_t kt = 0; kt < ktiles; kt += NS) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      if (s == 0 || kt + s < ktiles) {
        // Step 0 of tile kt + s (stage s), reading step 1 ahead.
        __builtin_amdgcn_sched_barrier(0);
        pipe_reads<OA, OB, TM, TN, WTM, WTN>(fa1, fb1, stages[s], 1, wm, wn, lane);
        pipe_mfma<TM, TN>(acc, fa0, fb0);
        mfma_then_reads<0, MF, NR, 2>();
        __builtin_amdgcn_sched_barrier(0);
        // Step 1: the next tile has landed here (NS - 3 younger tiles may be
        // in flight); after the barrier it has landed everywhere and no wave
        // reads the previous tile's stage, which is refilled with tile
        // kt + s + NS - 1.  Then step 0 of the next tile is read ahead (past
        // the last tile this reads a stage holding a reload, unused).
        wait_vmcnt<(NS - 3) * PER_TILE>();
        __builtin_amdgcn_s_barrier();
        // The next step's fragment reads and the refill's DMA instructions
        // are spread over the step's MFMAs -- one fragment read after each
        // MFMA, in the order the next step's MFMAs use them (A's first
        // fragment, B's, then A's others), and one DMA instruction after each
        // MFMA from the third -- so the MFMA pipe is not left idle while a
        // wave issues a burst of them and the first reads land well before
        // their use (0.75 -> 0.85 of the MFMA cycles in the main loop at
        // 4096^3); whatever the step has no MFMA left for follows it.
        char *refill = stages[(s + NS - 1) % NS];
        const auto sa = OA::template src_of<NW>(A, g.lda, m0, kclamp(kt + s + NS - 1), wave, lane);
        const auto sb = GN ? OB::template src_edge<NW>(B, g.ldb, n0, kbof(kt + s + NS - 1), wave, lane, brows)
                           : OB::template src_of<NW>(B, g.ldb, n0, kbof(kt + s + NS - 1), wave, lane);
        const char *nst = stages[(s + 1) % NS];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < MF || q < PER_TILE + 2 || q < TM + TN; ++q) {
          if (q < MF) {
            const int i = q / TN, j = q % TN;
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, fa1[i]),
                                                                __builtin_bit_cast(bf16x8, fb1[j]), acc[i][j], 0, 0, 0);
          }
          if (q == 0) fa0[0] = OA::frag(nst, wm * WTM, 0, lane);
          else if (q <= TN) fb0[q - 1] = OB::frag(nst + OA::BYTES, wn * WTN + (q - 1) * 32, 0, lane);
          else if (q < TN + TM) fa0[q - TN] = OA::frag(nst, wm * WTM + (q - TN) * 32, 0, lane);
          const int d = q - 2;
          if (d >= 0 && d < PA) OA::template issue<NW>(sa, d, refill, wave);
          else if (d >= PA && d < PER_TILE) OB::template issue<NW>(sb, d - PA, refill + OA::BYTES, wave);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
  }
  // No DMA may still be writing this workgroup's LDS when its waves end.
  wait_vmcnt<0>();

  // Fragment (i, j), value r: row 32 i + 8 (r / 4) + 4 (lane / 32) + r % 4,
  // column 32 j + lane % 32 of the wave's tile.  One base pointer per
  // fragment and 16 row offsets shared by all, so the addressing stays small
  // next to the accumulators.
  const int lrow = lane & 31, lhalf = lane >> 5;
  const int64_t row0 = m0 + wm * WTM + 4 * lhalf, col0 = n0 + wn * WTN + lrow;
  if constexpr (TN == 2) {
    if (g.qkv.mode) {
      __syncthreads();  // every wave past its last read of the stages
      if (n0 < static_cast<int64_t>(g.qkv.heads + g.qkv.kvh) * 64) {  // a tile with RoPE heads
        qkv_tables<BM, NS, STAGE, NW * 64>(g.qkv, m0, stages, tid);
        __syncthreads();
      }
      qkv_tail<TM, BM, STAGE / 256>(g, acc, row0, n0 + wn * WTN, lrow, m0, stages);
      return;
    }
  }
  if constexpr (TN % 2 == 0 && !GN) {
    if (g.swiglu) {
      // Fragments (i, 2 jp) and (i, 2 jp + 1) are the gate and up columns of
      // outputs (n0 + wn WTN) / 2 + 32 jp + lane % 32: silu(gate) * up as the
      // element-wise SILU_MUL computes it, stored in the asked form.
      uint16_t *P = static_cast<uint16_t *>(g.c);
      float *Pf = static_cast<float *>(g.c);
      const int64_t I = g.N / 2;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int jp = 0; jp < TN / 2; ++jp) {
          const int64_t oc = (n0 + wn * WTN) / 2 + 32 * jp + lrow;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int64_t row = row0 + i * 32 + 8 * (r >> 2) + (r & 3);
            const float gt = acc[i][2 * jp][r], up = acc[i][2 * jp + 1][r];
            const float y = swiglu_value(gt, up);
            if (g.swiglu == SWIGLU_PARTS) {
              uint16_t h, l;
              split_bf16(y, h, l);
              P[row * 2 * I + oc] = h;
              P[row * 2 * I + I + oc] = l;
            } else if (g.swiglu == SWIGLU_BF16) {
              P[row * I + oc] = f32_to_bf16_bits(y);
            } else {
              Pf[row * I + oc] = y;
            }
          }
        }
      }
      return;
    }
  }
  const bool plain = g.bias == nullptr && g.resid == nullptr;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      if (GN && col0 + j * 32 >= g.N) continue;
      TO *cij = C + (row0 + i * 32) * g.ldc + col0 + j * 32;
      float v[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) v[r] = acc[i][j][r];
      if (!plain) fragment_epilogue<false>(g, row0 + i * 32, col0 + j * 32, v);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int dr = 8 * (r >> 2) + (r & 3);
        if constexpr (sizeof(TO) == 2) cij[dr * g.ldc] = f32_to_bf16_bits(v[r]);
        else cij[dr * g.ldc] = v[r];
      }
    }
  }
}

// Two waves per SIMD (8 per workgroup): at most 256 registers a wave.
template <typename TO, int BM, int BN, int NS, bool AK, bool BKC, int WM, int WN, bool GN>
__global__ void __launch_bounds__(WM *WN * 64) gemm_pipe_kernel(GemmArgs g) {
  gemm_pipe_body<TO, BM, BN, NS, AK, BKC, WM, WN, GN>(g);
}

// One wave per SIMD (4 per workgroup): the whole 512-entry register file, so
// a 128 x 128 wave tile keeps its accumulators in the AGPRs.
template <typename TO, int BM, int BN, int NS, bool AK, bool BKC, int WM, int WN, bool GN>
__global__ void __launch_bounds__(WM *WN * 64) __attribute__((amdgpu_waves_per_eu(1, 1)))
gemm_pipe1_kernel(GemmArgs g) {
  gemm_pipe_body<TO, BM, BN, NS, AK, BKC, WM, WN, GN>(g);
}

// ------------------------------------------------- small-M products
// Decode-shaped products (M <= 8 rows of F32 activations against a
// k-contiguous weight, B stored [n, k]): the weight streams from HBM once,
// 16 bytes per lane per step, each wavefront owning GEMV_NR outputs for all
// M rows; lanes stride k and fold with a butterfly.  HBM-bound on the weight.
constexpr int GEMV_NR = 2;

__device__ __forceinline__ float gemv_wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

template <int M, typename SB, typename TO>
__global__ void __launch_bounds__(256) gemv_kernel(const float *A, int64_t lda, const SB *B, int64_t ldb, TO *C,
                                                   int64_t ldc, int64_t N, int64_t K, const float *bias,
                                                   const float *resid, int64_t ldr) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
  const int64_t n0 = wave * GEMV_NR;
  if (n0 >= N) return;
  float acc[M][GEMV_NR];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < GEMV_NR; ++r) acc[m][r] = 0.0f;
  for (int64_t k = static_cast<int64_t>(lane) * 8; k < K; k += 512) {
    float w[GEMV_NR][8];
#pragma unroll
    for (int r = 0; r < GEMV_NR; ++r) {
      if (n0 + r < N) {
        const SB *row = B + (n0 + r) * ldb + k;
        if constexpr (sizeof(SB) == 2) {
          const uint4 q = *reinterpret_cast<const uint4 *>(row);
          const uint32_t u[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            w[r][2 * e] = __uint_as_float(u[e] << 16);
            w[r][2 * e + 1] = __uint_as_float(u[e] & 0xffff0000u);
          }
        } else {
          const float4 q0 = *reinterpret_cast<const float4 *>(row);
          const float4 q1 = *reinterpret_cast<const float4 *>(row + 4);
          w[r][0] = q0.x; w[r][1] = q0.y; w[r][2] = q0.z; w[r][3] = q0.w;
          w[r][4] = q1.x; w[r][5] = q1.y; w[r][6] = q1.z; w[r][7] = q1.w;
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) w[r][e] = 0.0f;
      }
    }
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const float4 a0 = *reinterpret_cast<const float4 *>(A + m * lda + k);
      const float4 a1 = *reinterpret_cast<const float4 *>(A + m * lda + k + 4);
      const float av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
      for (int r = 0; r < GEMV_NR; ++r) {
        float t = acc[m][r];
#pragma unroll
        for (int e = 0; e < 8; ++e) t += av[e] * w[r][e];
        acc[m][r] = t;
      }
    }
  }
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < GEMV_NR; ++r) acc[m][r] = gemv_wave_sum(acc[m][r]);
  if (lane == 0) {
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int r = 0; r < GEMV_NR; ++r) {
        if (n0 + r < N) {
          float v = acc[m][r];
          if (bias) v = __fadd_rn(v, bias[n0 + r]);
          if (resid) v = __fadd_rn(resid[m * ldr + n0 + r], v);
          if constexpr (sizeof(TO) == 2) C[m * ldc + n0 + r] = f32_to_bf16_bits(v);
          else C[m * ldc + n0 + r] = v;
        }
      }
  }
}

// Split-K: the S partial products [S, M, N] added in slice order.
// The linear epilogue (bias over n, residual with row pitch ldr) applies to
// the sum.
template <typename TO>
__global__ void splitk_reduce(const float *part, int S, int64_t mn, int64_t n, TO *C, int64_t ldc, const float *bias,
                              const float *resid, int64_t ldr) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= mn) return;
  const int64_t row = i / n, col = i - row * n;
  // The epilogue operands and eight slices at a time requested before their
  // adds (in slice order), so the reduce is not one round trip per slice.
  const float bv = bias ? bias[col] : 0.0f, rv = resid ? resid[row * ldr + col] : 0.0f;
  float s = part[i];
  for (int z0 = 1; z0 < S; z0 += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (z0 + u < S) v[u] = part[(z0 + u) * mn + i];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (z0 + u < S) s += v[u];
  }
  if (bias) s = __fadd_rn(s, bv);
  if (resid) s = __fadd_rn(rv, s);
  if constexpr (sizeof(TO) == 2) C[row * ldc + col] = f32_to_bf16_bits(s);
  else C[row * ldc + col] = s;
}

// splitk_reduce then mi_rms_norm's row kernel in one pass, bit for bit the
// two: a wavefront a row, lane l owning columns l + 64 t; each value is the
// slices added in slice order, then the bias, then the residual (stored as
// the F32 result), and the row's sum of squares folds in the norm kernel's
// order before each value is divided by the RMS and scaled by the gain.
template <int T>
__global__ void __launch_bounds__(256) splitk_reduce_norm(const float *part, int S, int64_t M, int64_t n, float *C,
                                                          const float *bias, const float *resid, int64_t ldr,
                                                          const float *gamma, float eps, void *yn, int yn_elem) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const int64_t mn = M * n;
  // Every operand of the lane's columns is requested before the first add:
  // the slices four at a time across all columns (clamped addresses, so the
  // loads are unconditional), the gain, bias and residual with the first.
  float v[T], gm[T], bv[T], rv[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int64_t j = lane + 64 * t, jc = j < n ? j : n - 1, i = row * n + jc;
    v[t] = part[i];
    gm[t] = gamma ? gamma[jc] : 1.0f;
    bv[t] = bias ? bias[jc] : 0.0f;
    rv[t] = resid ? resid[row * ldr + jc] : 0.0f;
  }
  for (int z0 = 1; z0 < S; z0 += 4) {
    float p4[4][T];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const int64_t j = lane + 64 * t, jc = j < n ? j : n - 1;
        const int z = z0 + u < S ? z0 + u : S - 1;
        p4[u][t] = part[z * mn + row * n + jc];
      }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int t = 0; t < T; ++t)
        if (z0 + u < S) v[t] += p4[u][t];
  }
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int64_t j = lane + 64 * t;
    if (j < n) {
      float s = v[t];
      if (bias) s = __fadd_rn(s, bv[t]);
      if (resid) s = __fadd_rn(rv[t], s);
      v[t] = s;
      C[row * n + j] = s;
    } else {
      v[t] = 0.0f;
    }
  }
  float ss = 0.0f;
#pragma unroll
  for (int t = 0; t < T; ++t) ss += v[t] * v[t];
  ss = fold_sum<64>(ss);
  const float rms = __fsqrt_rn(ss / static_cast<float>(n) + eps);
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int64_t j = lane + 64 * t;
    if (j < n) {
      float y = v[t] / rms;
      if (gamma) y = y * gm[t];
      if (yn_elem == MI_BF16_PARTS) {
        uint16_t h, l;
        split_bf16(y, h, l);
        uint16_t *o = static_cast<uint16_t *>(yn) + 2 * row * n;
        o[j] = h;
        o[n + j] = l;
      } else if (yn_elem == MI_BF16) {
        static_cast<uint16_t *>(yn)[row * n + j] = f32_to_bf16_bits(y);
      } else {
        static_cast<float *>(yn)[row * n + j] = y;
      }
    }
  }
}

// ----------------------------------------------------------- launching
struct Plan {
  int64_t M, N, K, batch;
  bool ta, tb;
  int ea, eb, eo;  // element kinds
  const void *a, *b;
  void *c;
  int64_t sa, sb, sc;
  int64_t lda, ldb;   // row pitch of each operand's storage
  int64_t kc = 0;     // split-K slice length (register kernel only)
  int splits = 1;
  bool fast = true;   // F32 operands split into BF16 parts (the fast matmul mode)
  const float *bias = nullptr;   // linear epilogue (batch 1): C = resid + (A B + bias)
  const float *resid = nullptr;
  int64_t ldr = 0;
  int64_t ldc = 0;                // result row pitch (0: N)
  int64_t per_group = 0;          // items per group (0: one group of `batch`)
  int64_t sa2 = 0, sb2 = 0, sc2 = 0;  // group strides
  int64_t kb = 0;  // direct BF16 kernel: B's k extent when A's k repeats it (see GemmArgs)
  int swiglu = 0;  // direct BF16 kernel: gate|up pairs into silu(gate) * up (see GemmArgs)
  QkvTail qkv;     // direct BF16 kernel: the q|k|v tail (see QkvTail)
  // The RMSNorm of the F32 result's rows (mi_linear_add_rms_norm): taken by
  // the split-K reduce when the product splits over k (*norm_done set),
  // else run after the product by the caller.
  const float *norm_gamma = nullptr;
  float norm_eps = 0.0f;
  void *norm_out = nullptr;
  int norm_elem = MI_F32;
  bool *norm_done = nullptr;
};

template <typename T, typename SA, typename SB, typename TO, int BM, int BN, int WM, int WN, bool AK, bool BKC, bool GUARD,
          int STORE_AT = 3>
static hipError_t launch_cfg(const Plan &p, hipStream_t st) {
  constexpr int NT = WM * WN * 64;
  constexpr int SMEM = 2 * (BM + BN) * 128;
  auto kern = gemm_kernel<T, SA, SB, TO, BM, BN, WM, WN, AK, BKC, GUARD, STORE_AT>;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, SMEM);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  GemmArgs g;
  g.a = p.a; g.b = p.b; g.c = p.c;
  g.M = p.M; g.N = p.N; g.K = p.K;
  g.lda = p.lda;  // A is [m, k] or [k, m]
  g.ldb = p.ldb;  // B is [k, n] or [n, k]
  g.ldc = p.ldc > 0 ? p.ldc : p.N;
  g.sa = p.sa; g.sb = p.sb; g.sc = p.sc;
  g.per_group = p.per_group > 0 ? p.per_group : p.batch;
  g.sa2 = p.sa2; g.sb2 = p.sb2; g.sc2 = p.sc2;
  g.kc = p.kc;
  g.bias = p.bias; g.resid = p.resid; g.ldr = p.ldr;
  g.tiles_m = static_cast<int>((p.M + BM - 1) / BM);
  g.tiles_n = static_cast<int>((p.N + BN - 1) / BN);
  dim3 grid(static_cast<unsigned>(g.tiles_m * g.tiles_n), static_cast<unsigned>(p.batch),
            static_cast<unsigned>(p.splits));
  kern<<<grid, NT, SMEM, st>>>(g);
  return hipGetLastError();
}

template <typename TO, int BM, int BN, int NS, bool AK, bool BKC, int WM, int WN, bool GN>
static hipError_t launch_pipe_cfg(const Plan &p, hipStream_t st) {
  GemmArgs g;
  g.a = p.a; g.b = p.b; g.c = p.c;
  g.M = p.M; g.N = p.N; g.K = p.K;
  g.lda = p.lda;
  g.ldb = p.ldb;
  g.ldc = p.ldc > 0 ? p.ldc : p.N;
  g.sa = p.sa; g.sb = p.sb; g.sc = p.sc;
  g.per_group = p.per_group > 0 ? p.per_group : p.batch;
  g.sa2 = p.sa2; g.sb2 = p.sb2; g.sc2 = p.sc2;
  g.kc = 0;
  g.bias = p.bias; g.resid = p.resid; g.ldr = p.ldr;
  g.kb = p.kb;
  g.swiglu = p.swiglu;
  g.qkv = p.qkv;
  g.tiles_m = static_cast<int>(p.M / BM);
  g.tiles_n = static_cast<int>((p.N + BN - 1) / BN);
  dim3 grid(static_cast<unsigned>(g.tiles_m * g.tiles_n), static_cast<unsigned>(p.batch));
  if constexpr (WM * WN == 4) gemm_pipe1_kernel<TO, BM, BN, NS, AK, BKC, WM, WN, GN><<<grid, 256, 0, st>>>(g);
  else gemm_pipe_kernel<TO, BM, BN, NS, AK, BKC, WM, WN, GN><<<grid, WM * WN * 64, 0, st>>>(g);
  return hipGetLastError();
}

template <typename TO, int BM, int BN, int NS, int WM, int WN>
static hipError_t launch_pipe(const Plan &p, hipStream_t st) {
  const bool ak = !p.ta, bk = p.tb;
  if (ak && bk) return launch_pipe_cfg<TO, BM, BN, NS, true, true, WM, WN, false>(p, st);
  if (ak && !bk) return launch_pipe_cfg<TO, BM, BN, NS, true, false, WM, WN, false>(p, st);
  if (!ak && bk) return launch_pipe_cfg<TO, BM, BN, NS, false, true, WM, WN, false>(p, st);
  return launch_pipe_cfg<TO, BM, BN, NS, false, false, WM, WN, false>(p, st);
}

// A width that is not a multiple of the tile: B k-contiguous ([N, K] as the
// weights are stored), N a multiple of 16, A k-contiguous.
template <typename TO, int BM, int BN, int NS, int WM, int WN>
static hipError_t launch_pipe_edge(const Plan &p, hipStream_t st) {
  return launch_pipe_cfg<TO, BM, BN, NS, true, true, WM, WN, true>(p, st);
}


// Operand orientation: A k-contiguous unless transposed; B k-contiguous when transposed.
template <typename T, typename SA, typename SB, typename TO, int BM, int BN, int WM, int WN, bool GUARD>
static hipError_t launch_orient(const Plan &p, hipStream_t st) {
  const bool ak = !p.ta, bk = p.tb;
  if (ak && bk) return launch_cfg<T, SA, SB, TO, BM, BN, WM, WN, true, true, GUARD>(p, st);
  if (ak && !bk) return launch_cfg<T, SA, SB, TO, BM, BN, WM, WN, true, false, GUARD>(p, st);
  if (!ak && bk) return launch_cfg<T, SA, SB, TO, BM, BN, WM, WN, false, true, GUARD>(p, st);
  return launch_cfg<T, SA, SB, TO, BM, BN, WM, WN, false, false, GUARD>(p, st);
}

// Every operand pointer, leading dimension and batch stride a multiple of the
// 16-byte chunk, and the shape a multiple of the tile: the unguarded kernel.
static bool tiles_exactly(const Plan &p, int bm, int bn, int bk, int64_t align_elems) {
  if (p.M % bm || p.N % bn || p.K % bk) return false;
  const int64_t lda = p.lda, ldb = p.ldb;
  if (lda % align_elems || ldb % align_elems) return false;
  if (p.sa % align_elems || p.sb % align_elems || p.sa2 % align_elems || p.sb2 % align_elems) return false;
  if ((reinterpret_cast<uintptr_t>(p.a) & 15) || (reinterpret_cast<uintptr_t>(p.b) & 15)) return false;
  return true;
}

template <typename SA, typename SB, typename TO, int BM, int BN, int WM, int WN, bool AK, bool BKC, bool GUARD>
static hipError_t launch_split_cfg(const Plan &p, hipStream_t st) {
  constexpr int NT = WM * WN * 64;
  constexpr int SMEM = 2 * (BM * 128 * (sizeof(SA) == 4 ? 2 : 1) + BN * 128 * (sizeof(SB) == 4 ? 2 : 1));
  auto kern = gemm_split_kernel<SA, SB, TO, BM, BN, WM, WN, AK, BKC, GUARD>;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, SMEM);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  GemmArgs g;
  g.a = p.a; g.b = p.b; g.c = p.c;
  g.M = p.M; g.N = p.N; g.K = p.K;
  g.lda = p.lda;
  g.ldb = p.ldb;
  g.ldc = p.ldc > 0 ? p.ldc : p.N;
  g.sa = p.sa; g.sb = p.sb; g.sc = p.sc;
  g.per_group = p.per_group > 0 ? p.per_group : p.batch;
  g.sa2 = p.sa2; g.sb2 = p.sb2; g.sc2 = p.sc2;
  g.kc = p.kc;
  g.bias = p.bias; g.resid = p.resid; g.ldr = p.ldr;
  g.tiles_m = static_cast<int>((p.M + BM - 1) / BM);
  g.tiles_n = static_cast<int>((p.N + BN - 1) / BN);
  dim3 grid(static_cast<unsigned>(g.tiles_m * g.tiles_n), static_cast<unsigned>(p.batch),
            static_cast<unsigned>(p.splits));
  kern<<<grid, NT, SMEM, st>>>(g);
  return hipGetLastError();
}

template <typename SA, typename SB, typename TO, int BM, int BN, int WM, int WN, bool GUARD>
static hipError_t launch_split_orient(const Plan &p, hipStream_t st) {
  const bool ak = !p.ta, bk = p.tb;
  if (ak && bk) return launch_split_cfg<SA, SB, TO, BM, BN, WM, WN, true, true, GUARD>(p, st);
  if (ak && !bk) return launch_split_cfg<SA, SB, TO, BM, BN, WM, WN, true, false, GUARD>(p, st);
  if (!ak && bk) return launch_split_cfg<SA, SB, TO, BM, BN, WM, WN, false, true, GUARD>(p, st);
  return launch_split_cfg<SA, SB, TO, BM, BN, WM, WN, false, false, GUARD>(p, st);
}

// Columns [n0, n0 + n) of a single product (no batch, no split-K) as a plan
// of its own: B, the result, the bias and the residual start n0 columns in,
// the result and residual keep their full row pitch.
static Plan column_block(const Plan &p, int64_t n0, int64_t n) {
  Plan q = p;
  const size_t esb = p.eb == MI_BF16 ? 2 : 4, eso = p.eo == MI_BF16 ? 2 : 4;
  q.N = n;
  q.b = static_cast<const char *>(p.b) + static_cast<size_t>(p.tb ? n0 * p.ldb : n0) * esb;
  q.c = static_cast<char *>(p.c) + static_cast<size_t>(n0) * eso;
  q.ldc = p.ldc > 0 ? p.ldc : p.N;
  if (p.bias) q.bias = p.bias + n0;
  if (p.resid) q.resid = p.resid + n0;
  return q;
}

// F32 (or mixed) operands in the fast mode: the split kernel, 128 x 128 tiles
// when they give every CU a tile, else 64 x 64.  A width that is not a
// multiple of 128 (a 960-wide q|k|v or 576-wide down projection) runs its
// 128-aligned columns on unguarded tiles and only the rest on the guarded
// form: the guarded loads slow every tile, not just the edge ones (a
// 16384 x 960 x 576 product 257 us guarded against 251 us for an exact one
// three times its size).
template <typename SA, typename SB, typename TO>
static hipError_t run_split(const Plan &p, hipStream_t st) {
  const int64_t tiles128 = ((p.M + 127) / 128) * ((p.N + 127) / 128) * p.batch;
  if (tiles128 >= 256) {
    if (tiles_exactly(p, 128, 128, 64, 8)) return launch_split_orient<SA, SB, TO, 128, 128, 2, 2, false>(p, st);
    if (p.batch == 1 && p.kc == 0 && p.N > 128) {
      const int64_t ni = p.N / 128 * 128;
      const Plan in = column_block(p, 0, ni), edge = column_block(p, ni, p.N - ni);
      if (tiles_exactly(in, 128, 128, 64, 8)) {
        hipError_t e = launch_split_orient<SA, SB, TO, 128, 128, 2, 2, false>(in, st);
        if (e != hipSuccess) return e;
        if (tiles_exactly(edge, 64, 64, 64, 8)) return launch_split_orient<SA, SB, TO, 64, 64, 2, 2, false>(edge, st);
        return launch_split_orient<SA, SB, TO, 64, 64, 2, 2, true>(edge, st);
      }
    }
    return launch_split_orient<SA, SB, TO, 128, 128, 2, 2, true>(p, st);
  }
  if (tiles_exactly(p, 64, 64, 64, 8)) return launch_split_orient<SA, SB, TO, 64, 64, 2, 2, false>(p, st);
  return launch_split_orient<SA, SB, TO, 64, 64, 2, 2, true>(p, st);
}

static bool parts_small_tiles(const Plan &p);

// A width of 192s that 256 does not divide (576: a 576-wide model's o and
// down products), plain or with bias and residual, A and B k-contiguous, at
// most a tile a CU: 256 x 192 tiles, eight waves of 64 x 96, where 256 x 256
// ones would leave a quarter of every third column tile unused.  The q|k|v
// and gate|up tails take column pairs of the 64-wide wave tiles, so those
// keep the 256-wide ones.
static bool pipe_192_fits(const Plan &p) {
  return p.batch == 1 && !p.ta && p.tb && p.N % 256 && p.N % 192 == 0 && p.M % 256 == 0 && p.K % 32 == 0 &&
         (p.M / 256) * (p.N / 192) <= 256 &&
         p.lda % 8 == 0 && p.ldb % 8 == 0 && !(reinterpret_cast<uintptr_t>(p.a) & 15) &&
         !(reinterpret_cast<uintptr_t>(p.b) & 15) && !p.swiglu && !p.qkv.mode;
}

template <typename TO>
static hipError_t run_bf16(const Plan &p, hipStream_t st) {
  using T = uint16_t;
  auto tiles = [&](int64_t bm, int64_t bn) { return ((p.M + bm - 1) / bm) * ((p.N + bn - 1) / bn) * p.batch; };
  // Exactly tiled shapes take the pipelined direct HBM -> LDS kernel: 256 x
  // 256 tiles (8 waves of 128 x 64, two per SIMD) when they give most of the
  // 256 CUs a tile, else 128 x 128 tiles (4 waves of 64 x 64) from 16 tiles
  // up (512^3 in 7.5 us against 8.9 on 64 x 64 register tiles); five LDS
  // stages of k 32 either way.
  if (tiles_exactly(p, 256, 256, 32, 8) && tiles(256, 256) >= 192) return launch_pipe<TO, 256, 256, 5, 2, 4>(p, st);
  if (tiles_exactly(p, 128, 128, 32, 8) && tiles(128, 128) >= 16) return launch_pipe<TO, 128, 128, 5, 2, 2>(p, st);
  // Widths of 16s that the tiles do not divide, against a k-contiguous B (a
  // weight stored [n, k]): the direct kernel's edge tiles, where its rows and
  // k tile, over at least 128 tiles of 128 x 128 (a batch-32 prefill's o,
  // down and q|k|v products at 576 and 960 columns: the performance-contract
  // prefill 12.1 -> 11.3 ms; at 512 rows the 64 x 64 register tiles stay
  // ahead, 2.36 against 2.56 ms for that prefill).
  if (p.batch == 1 && !p.ta && p.tb && p.N % 16 == 0 && p.M % 128 == 0 && p.K % 32 == 0 && p.lda % 8 == 0 &&
      p.ldb % 8 == 0 && !(reinterpret_cast<uintptr_t>(p.a) & 15) && !(reinterpret_cast<uintptr_t>(p.b) & 15) &&
      tiles(128, 128) >= 128) {
    if (!parts_small_tiles(p)) {
      if (pipe_192_fits(p)) return launch_pipe_cfg<TO, 256, 192, 5, true, true, 4, 2, false>(p, st);
      return launch_pipe_edge<TO, 256, 256, 5, 2, 4>(p, st);
    }
    return launch_pipe_edge<TO, 128, 128, 5, 2, 2>(p, st);
  }
  if (tiles_exactly(p, 64, 64, 64, 8))
    return launch_orient<T, T, T, TO, 64, 64, 2, 2, false>(p, st);
  return launch_orient<T, T, T, TO, 64, 64, 2, 2, true>(p, st);
}

template <typename SA, typename SB, typename TO>
static hipError_t run_f32(const Plan &p, hipStream_t st) {
  using T = float;
  const int64_t al = (sizeof(SA) == 2 || sizeof(SB) == 2) ? 4 : 4;
  // 128 x 128 tiles once they fill every CU; below that 64 x 64 tiles (four
  // times the blocks) finish first -- e.g. a [256, 8192] product over k 2048
  // in 117 us against 167 us on 128 tiles of 128 x 128.
  const int64_t tiles128 = ((p.M + 127) / 128) * ((p.N + 127) / 128) * p.batch;
  if (tiles128 >= 256 && tiles_exactly(p, 128, 128, 32, al))
    return launch_orient<T, SA, SB, TO, 128, 128, 2, 2, false>(p, st);
  if (tiles_exactly(p, 64, 64, 32, al))
    return launch_orient<T, SA, SB, TO, 64, 64, 2, 2, false>(p, st);
  return launch_orient<T, SA, SB, TO, 64, 64, 2, 2, true>(p, st);
}

static hipError_t run_plan(const Plan &p, hipStream_t st) {
  const bool bf = p.eo == MI_BF16;
  if (p.ea == MI_BF16 && p.eb == MI_BF16)
    return bf ? run_bf16<uint16_t>(p, st) : run_bf16<float>(p, st);
  // The fast mode splits F32 operands where the product is large enough to be
  // bound by the matrix cores (at least 2^33 multiply-adds over at least 128
  // tiles of 128 x 128): below that the kernels are bound by load latency and
  // the split's conversions only add work, so the F32 kernel runs (more
  // accurate, and faster there).
  // F32 activations against BF16 weights over at least 256 rows are the
  // exception at any size: split, only the activations take two BF16 parts,
  // and the k loop runs on the BF16 matrix cores instead of the F32 ones (a
  // 512-token prefill of the SmolLM2-shaped decoder 8.7 -> 7.5 ms; its
  // products at 2048 - 8192 rows, us: gate|up at 2048 rows 86.6 -> 42.0, down
  // at 4096 98.7 -> 39.8, down at 8192 167.7 -> 81.7, o at 8192 66.9 -> 38.0).
  const int64_t macs = p.M * p.N * p.K * p.batch;
  const bool split_pays =
      (macs >= (int64_t(1) << 33) && ((p.M + 127) / 128) * ((p.N + 127) / 128) * p.batch >= 128) ||
      (p.ea == MI_F32 && p.eb == MI_BF16 && p.M >= 256);
  if (p.fast && split_pays) {
    if (p.ea == MI_F32 && p.eb == MI_F32)
      return bf ? run_split<float, float, uint16_t>(p, st) : run_split<float, float, float>(p, st);
    if (p.ea == MI_F32)
      return bf ? run_split<float, uint16_t, uint16_t>(p, st) : run_split<float, uint16_t, float>(p, st);
    return bf ? run_split<uint16_t, float, uint16_t>(p, st) : run_split<uint16_t, float, float>(p, st);
  }
  if (p.ea == MI_F32 && p.eb == MI_F32)
    return bf ? run_f32<float, float, uint16_t>(p, st) : run_f32<float, float, float>(p, st);
  if (p.ea == MI_F32 && p.eb == MI_BF16)
    return bf ? run_f32<float, uint16_t, uint16_t>(p, st) : run_f32<float, uint16_t, float>(p, st);
  return bf ? run_f32<uint16_t, float, uint16_t>(p, st) : run_f32<uint16_t, float, float>(p, st);
}

}  // namespace mi

using namespace mi;

namespace mi {

template <int M>
static void launch_gemv_m(const Plan &p, hipStream_t st) {
  const unsigned grid = static_cast<unsigned>((p.N + 4 * GEMV_NR - 1) / (4 * GEMV_NR));
  const float *A = static_cast<const float *>(p.a);
  if (p.eb == MI_BF16) {
    const uint16_t *B = static_cast<const uint16_t *>(p.b);
    if (p.eo == MI_BF16) gemv_kernel<M, uint16_t, uint16_t><<<grid, 256, 0, st>>>(A, p.lda, B, p.ldb, static_cast<uint16_t *>(p.c), p.ldc > 0 ? p.ldc : p.N, p.N, p.K, p.bias,
                                                                  p.resid, p.ldr);
    else gemv_kernel<M, uint16_t, float><<<grid, 256, 0, st>>>(A, p.lda, B, p.ldb, static_cast<float *>(p.c), p.ldc > 0 ? p.ldc : p.N, p.N, p.K, p.bias,
                                                                  p.resid, p.ldr);
  } else {
    const float *B = static_cast<const float *>(p.b);
    if (p.eo == MI_BF16) gemv_kernel<M, float, uint16_t><<<grid, 256, 0, st>>>(A, p.lda, B, p.ldb, static_cast<uint16_t *>(p.c), p.ldc > 0 ? p.ldc : p.N, p.N, p.K, p.bias,
                                                                  p.resid, p.ldr);
    else gemv_kernel<M, float, float><<<grid, 256, 0, st>>>(A, p.lda, B, p.ldb, static_cast<float *>(p.c), p.ldc > 0 ? p.ldc : p.N, p.N, p.K, p.bias,
                                                                  p.resid, p.ldr);
  }
}

// The GEMV applies: a few F32 rows against a k-contiguous F32 or BF16
// weight, 16-byte aligned rows.
static bool gemv_fits(const Plan &p) {
  if (p.batch != 1 || p.M < 1 || p.M > 8 || !p.tb || p.ta || p.ea != MI_F32) return false;
  if (p.K % 8 || p.lda % 4 || p.ldb % 8) return false;
  if ((reinterpret_cast<uintptr_t>(p.a) & 15) || (reinterpret_cast<uintptr_t>(p.b) & 15)) return false;
  return true;
}

static void launch_gemv(const Plan &p, hipStream_t st) {
  // One instantiation per row count: a kernel never touches a row past M.
  switch (p.M) {
    case 1: launch_gemv_m<1>(p, st); break;
    case 2: launch_gemv_m<2>(p, st); break;
    case 3: launch_gemv_m<3>(p, st); break;
    case 4: launch_gemv_m<4>(p, st); break;
    case 5: launch_gemv_m<5>(p, st); break;
    case 6: launch_gemv_m<6>(p, st); break;
    case 7: launch_gemv_m<7>(p, st); break;
    default: launch_gemv_m<8>(p, st); break;  // gemv_fits admits M <= 8 only
  }
}

// Whether a sliced product runs on the split kernel: F32 activations (256 or
// more rows) against a BF16 weight in the fast mode.
static bool split_slices(const Plan &p) {
  return p.fast && p.ea == MI_F32 && p.eb == MI_BF16 && p.M >= 256;
}

// Split-K for few output tiles over a long k: enough (tile, slice) pairs to
// give most CUs work.  Measured on the training steps' products: with 64 or
// more tiles, slicing a k below 1024 costs more (the reduce launch) than it
// gains and slices of 256 suit k = 1024; k >= 2048, or a handful of tiles,
// takes slices down to 128 (a [256, 256] x k 2048 product: 72 us unsliced,
// 16 us in 16 slices; the MLP's [64, 784] x [784, 128] gains from 6).
static int splitk_slices(const Plan &p) {
  if (p.batch != 1) return 1;
  // BF16 operands tiled exactly by 128 run the pipelined kernel whole once
  // its tiles (16 or more) cover the k loop, tiles x 128 >= k: 1024^3 in
  // 11 us against 26 us split four ways on the register kernel, 768 x 768
  // over k 2048 in 18 against 26; 512 x 512 over k 4096 stays split (27 us
  // against 32).
  if (p.ea == MI_BF16 && p.eb == MI_BF16 && tiles_exactly(p, 128, 128, 32, 8)) {
    const int64_t t128 = (p.M / 128) * (p.N / 128);
    if (t128 >= 16 && t128 * 128 >= p.K) return 1;
  }
  const int64_t tiles = ((p.M + 63) / 64) * ((p.N + 63) / 64);
  if (tiles >= 512 || p.K < 256) return 1;
  // Those on the split kernel slice from k 512 under 128 tiles (a 512-token
  // prefill's o, q|k|v and down products: batch 1 3.25 -> 3.01 ms).
  if (split_slices(p) && p.K >= 512 && tiles < 128) return p.K >= 1024 ? 4 : 2;
  if (p.K < 1024 && tiles >= 64) return 1;
  int64_t s = (1024 + tiles - 1) / tiles;
  const int64_t smax = (p.K >= 2048 || tiles < 64) ? p.K / 128 : p.K / 256;
  if (s > smax) s = smax;
  if (s > 32) s = 32;
  return s < 2 ? 1 : static_cast<int>(s);
}

// Slices are multiples of 64 long, so with m and n multiples of 64 and k of
// 32 every slice tiles exactly and the unguarded loads run.
template <typename T, typename SA, typename SB>
static hipError_t run_splitk_kernels(const Plan &p, hipStream_t st) {
  if (tiles_exactly(p, 64, 64, 32, 4)) return launch_orient<T, SA, SB, float, 64, 64, 2, 2, false>(p, st);
  return launch_orient<T, SA, SB, float, 64, 64, 2, 2, true>(p, st);
}

// Slice length (on k-tile boundaries of both precisions) and the slice count
// it gives for p.splits requested slices.
static void plan_slices(Plan &p) {
  const int S = p.splits;
  const int64_t align = 64;
  p.kc = ((p.K + S - 1) / S + align - 1) / align * align;
  p.splits = static_cast<int>((p.K + p.kc - 1) / p.kc);
}

// The slices' raw partial products, [S, M, N] packed at part.
static hipError_t run_slices(const Plan &p, float *part, hipStream_t st) {
  Plan q = p;
  q.c = part;
  q.eo = MI_F32;
  q.bias = q.resid = nullptr;
  q.ldc = 0;
  // F32 activations against a BF16 weight in the fast mode: the slices on
  // the split kernel (activations in two BF16 parts on the BF16 matrix
  // cores), as the unsliced product runs.
  if (split_slices(q)) return run_split<float, uint16_t, float>(q, st);
  if (q.ea == MI_BF16 && q.eb == MI_BF16) return run_splitk_kernels<uint16_t, uint16_t, uint16_t>(q, st);
  if (q.ea == MI_F32 && q.eb == MI_F32) return run_splitk_kernels<float, float, float>(q, st);
  if (q.ea == MI_F32) return run_splitk_kernels<float, float, uint16_t>(q, st);
  return run_splitk_kernels<float, uint16_t, float>(q, st);
}

static hipError_t run_splitk(Plan p, float *part, hipStream_t st) {
  plan_slices(p);
  void *final_c = p.c;
  const int eo = p.eo;
  const float *bias = p.bias, *resid = p.resid;
  const int64_t ldc = p.ldc > 0 ? p.ldc : p.N;
  hipError_t e = run_slices(p, part, st);
  if (e != hipSuccess) return e;
  const int64_t mn = p.M * p.N;
  const unsigned g = static_cast<unsigned>((mn + 255) / 256);
  if (p.norm_out && eo == MI_F32 && ldc == p.N && p.N <= 2048 && p.batch == 1) {
    const unsigned gr = static_cast<unsigned>((p.M + 3) / 4);
    float *y = static_cast<float *>(final_c);
    const int64_t n = p.N;
#define MI_SRN(T) splitk_reduce_norm<T><<<gr, 256, 0, st>>>(part, p.splits, p.M, n, y, bias, resid, p.ldr, \
                                                            p.norm_gamma, p.norm_eps, p.norm_out, p.norm_elem)
    // T = ceil(n / 64) where instantiated (576, 768, 960, 1536 columns: 9,
    // 12, 15, 24), else the next size up: no lane loads padded columns.
    const int64_t t = (n + 63) / 64;
    if (t <= 1) MI_SRN(1);
    else if (t <= 2) MI_SRN(2);
    else if (t <= 4) MI_SRN(4);
    else if (t <= 8) MI_SRN(8);
    else if (t <= 9) MI_SRN(9);
    else if (t <= 12) MI_SRN(12);
    else if (t <= 15) MI_SRN(15);
    else if (t <= 16) MI_SRN(16);
    else if (t <= 24) MI_SRN(24);
    else MI_SRN(32);
#undef MI_SRN
    if (p.norm_done) *p.norm_done = true;
    return hipGetLastError();
  }
  if (eo == MI_BF16)
    splitk_reduce<uint16_t><<<g, 256, 0, st>>>(part, p.splits, mn, p.N, static_cast<uint16_t *>(final_c), ldc, bias,
                                                resid, p.ldr);
  else
    splitk_reduce<float><<<g, 256, 0, st>>>(part, p.splits, mn, p.N, static_cast<float *>(final_c), ldc, bias, resid,
                                             p.ldr);
  return hipGetLastError();
}

// Check that `rows x cols` items at off + i * stride (row pitch ld) lie in x.
static bool items_in(const Buffer *x, int64_t batch, int64_t rows, int64_t cols, int64_t off, int64_t stride,
                     int64_t ld) {
  if (rows == 0 || cols == 0) return true;
  if (off < 0 || cols > ld || ld != x->cols) return false;
  const int64_t last = off + (batch - 1) * (stride > 0 ? stride : 0) + (rows - 1) * ld + cols - 1;
  return last < x->numel() && (stride >= 0);
}

// Check that item (g, i) of groups x per_group, `rows x cols` at
// at[0] + g * at[1] + i * at[2] with row pitch x->cols, lies in x for all g, i.
static bool grouped_items_in(const Buffer *x, int64_t groups, int64_t per_group, int64_t rows, int64_t cols,
                             const int64_t *at) {
  const int64_t n = x->numel(), ld = x->cols;
  if (at[0] < 0 || at[1] < 0 || at[2] < 0 || at[1] > n || at[2] > n || cols > ld) return false;
  const int64_t last = at[0] + (groups - 1) * at[1] + (per_group - 1) * at[2] + (rows - 1) * ld + cols - 1;
  return last < n;
}

// Launch a planned product (M, N, K >= 1) into p.c: the GEMV for a few rows
// against a k-contiguous weight, split-K for few tiles over a long k, else
// the tiled kernels.
// F32 rows [M, K] -> BF16 [M, 2 K]: each row's hi parts then its lo parts
// (split_bf16), eight elements a thread.
__global__ void __launch_bounds__(256) split_rows_kernel(const float *a, int64_t lda, uint16_t *out, int64_t M,
                                                         int64_t K) {
  const int64_t per_row = K / 8;
  const int64_t n = M * per_row;
  for (int64_t u = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; u < n;
       u += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t r = u / per_row, c = (u - r * per_row) * 8;
    const float4 v0 = *reinterpret_cast<const float4 *>(a + r * lda + c);
    const float4 v1 = *reinterpret_cast<const float4 *>(a + r * lda + c + 4);
    const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    uint4 hv, lv;
    split_bf16x2(v[0], v[1], hv.x, lv.x);
    split_bf16x2(v[2], v[3], hv.y, lv.y);
    split_bf16x2(v[4], v[5], hv.z, lv.z);
    split_bf16x2(v[6], v[7], hv.w, lv.w);
    *reinterpret_cast<uint4 *>(out + r * 2 * K + c) = hv;
    *reinterpret_cast<uint4 *>(out + r * 2 * K + K + c) = lv;
  }
}

// The fast mode's F32 x BF16 product as one BF16 product on the direct
// kernel: A's rows split once into their BF16 hi and lo parts, side by side
// ([M, 2 K]: A = hi + lo to 2^-17 relative, the same split the split kernel
// makes in registers), against B whose k wraps every K -- so the k loop
// accumulates hi . b then lo . b in F32.  The split costs one pass over A;
// the product then runs at the BF16 kernel's rate instead of the split
// kernel's (whose per-tile conversions hold it to a fraction of it).  For
// products big enough to fill the chip with 256 x 256 tiles.
static bool parts_direct_fits(const Plan &p);
static bool stacked_split_pays(const Plan &p) {
  if (!p.fast || p.ea != MI_F32 || p.kc != 0 || p.lda % 4 || (reinterpret_cast<uintptr_t>(p.a) & 15)) return false;
  if (p.M % 256 || !parts_direct_fits(p)) return false;
  const int64_t tiles = (p.M / 256) * ((p.N + 255) / 256);
  return tiles >= 128 && p.M * p.N * p.K >= (int64_t(1) << 32);
}

// Whether the direct kernel takes an F32 x BF16 product of plan p from A's
// parts: rows in 128-row tiles (256-row tiles where they fill the chip),
// whole k-tiles on each side of the wrap, B's width a multiple of the tile or
// (k-contiguous B) of 16 for the edge tiles.
static bool parts_direct_fits(const Plan &p) {
  if (p.eb != MI_BF16 || p.ta || p.batch != 1 || p.K % 32 || p.M % 128) return false;
  if ((reinterpret_cast<uintptr_t>(p.b) & 15) || p.ldb % 8) return false;
  if (p.M % 256 && p.N % 128 && !p.tb) return false;
  return p.N % 256 == 0 || (p.tb && p.N % 16 == 0) || (p.M % 256 && p.N % 128 == 0);
}

// Products of fewer than 192 tiles of 256 x 256 (or 128-row multiples) take
// the 128 x 128 tiles.
static bool parts_small_tiles(const Plan &p) {
  return p.M % 256 || (p.M / 256) * ((p.N + 255) / 256) < 192;
}

// The product of plan p (A F32 [M, K]) from A's parts at `parts` ([M, 2 K]
// BF16: each row's heads, then its remainders) on the direct kernel, B's k
// wrapping every K.
// A BF16 x BF16 product on the direct kernel, tiled as parts_small_tiles
// and parts_direct_fits plan it.
static hipError_t launch_direct(const Plan &q, hipStream_t st) {
  const bool bf = q.eo == MI_BF16;
  if (parts_small_tiles(q)) {
    if (q.N % 128 == 0)
      return bf ? launch_pipe<uint16_t, 128, 128, 5, 2, 2>(q, st) : launch_pipe<float, 128, 128, 5, 2, 2>(q, st);
    return bf ? launch_pipe_edge<uint16_t, 128, 128, 5, 2, 2>(q, st) : launch_pipe_edge<float, 128, 128, 5, 2, 2>(q, st);
  }
  if (q.N % 256 == 0)
    return bf ? launch_pipe<uint16_t, 256, 256, 5, 2, 4>(q, st) : launch_pipe<float, 256, 256, 5, 2, 4>(q, st);
  if (pipe_192_fits(q))
    return bf ? launch_pipe_cfg<uint16_t, 256, 192, 5, true, true, 4, 2, false>(q, st)
              : launch_pipe_cfg<float, 256, 192, 5, true, true, 4, 2, false>(q, st);
  return bf ? launch_pipe_edge<uint16_t, 256, 256, 5, 2, 4>(q, st) : launch_pipe_edge<float, 256, 256, 5, 2, 4>(q, st);
}

static hipError_t launch_parts(const Plan &p, const void *parts, hipStream_t st) {
  Plan q = p;
  q.a = parts;
  q.ea = MI_BF16;
  q.lda = 2 * p.K;
  q.K = 2 * p.K;
  q.kb = p.K;
  return launch_direct(q, st);
}

static int run_stacked_split(mi_ctx *ctx, const Plan &p) {
  mi_id tid;
  Buffer *tb;
  int s = new_buffer(ctx, p.M, 2 * p.K, MI_BF16, &tid, &tb);
  if (s) return s;
  const int64_t units = p.M * (p.K / 8);
  const unsigned g = static_cast<unsigned>(units / 256 + 1 < 65536 ? units / 256 + 1 : 65536);
  split_rows_kernel<<<g, 256, 0, ctx->stream>>>(static_cast<const float *>(p.a), p.lda,
                                                static_cast<uint16_t *>(tb->ptr), p.M, p.K);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) e = launch_parts(p, tb->ptr, ctx->stream);
  mi_free(ctx, tid);  // stream-ordered: the block is reused only by later work
  if (e != hipSuccess) return fail(ctx, MI_E_HIP, "matmul launch: %s", hipGetErrorString(e));
  return check_launch(ctx, "matmul");
}

static int run_product(mi_ctx *ctx, Plan &p) {
  hipError_t e;
  if (stacked_split_pays(p)) return run_stacked_split(ctx, p);
  if (gemv_fits(p)) {
    launch_gemv(p, ctx->stream);
    e = hipGetLastError();
  } else if ((p.splits = splitk_slices(p)) > 1) {
    float *part = static_cast<float *>(scratch(ctx, static_cast<size_t>(p.splits) * p.M * p.N * sizeof(float)));
    if (!part) return fail(ctx, MI_E_OOM, "split-K scratch");
    e = run_splitk(p, part, ctx->stream);
  } else {
    p.splits = 1;
    e = run_plan(p, ctx->stream);
  }
  if (e != hipSuccess) return fail(ctx, MI_E_HIP, "matmul launch: %s", hipGetErrorString(e));
  return check_launch(ctx, "matmul");
}

}  // namespace mi

// The epilogue operands of mi_linear (absent for plain products).
struct LinearTerms {
  const float *bias = nullptr;
  const float *resid = nullptr;
  int64_t ldr = 0;
  // mi_linear_add_rms_norm: the result rows' RMSNorm into norm_out (see Plan).
  const float *norm_gamma = nullptr;
  float norm_eps = 0.0f;
  void *norm_out = nullptr;
  int norm_elem = MI_F32;
  bool *norm_done = nullptr;
};

static int matmul_common(mi_ctx *ctx, mi_id a, int ta, mi_id b, int tb, int64_t batch, int64_t m, int64_t k,
                         int64_t n, int mode, const int64_t *blk, int out_elem, mi_id *out,
                         const LinearTerms &lin = LinearTerms()) {
  // mode 0: plain; 1: stacked batch; 2: explicit item offsets/strides (blk =
  // {a_off, a_stride, b_off, b_stride}), items read with the operand's row pitch.
  if (!out) return fail(ctx, MI_E_ARG, "null out pointer");
  MI_BUF(ctx, A, a);
  MI_BUF(ctx, B, b);
  if (!elem_float(A->elem) || !elem_float(B->elem))
    return fail(ctx, MI_E_ARG, "matmul of %s and %s", elem_name(A->elem), elem_name(B->elem));
  if (A->tiles || B->tiles) return fail(ctx, MI_E_ARG, "matmul of an operand in tiles (mi_linear reads them)");
  if (out_elem != MI_F32 && out_elem != MI_BF16) return fail(ctx, MI_E_ARG, "matmul result kind %s", elem_name(out_elem));
  Plan p;
  p.ta = ta != 0; p.tb = tb != 0;
  p.fast = ctx->matmul_mode == MI_MATMUL_FAST;
  p.ea = A->elem; p.eb = B->elem; p.eo = out_elem;
  p.a = A->ptr; p.b = B->ptr;
  if (mode == 0) {
    p.M = ta ? A->cols : A->rows;
    p.K = ta ? A->rows : A->cols;
    const int64_t kb = tb ? B->cols : B->rows;
    p.N = tb ? B->rows : B->cols;
    if (kb != p.K)
      return fail(ctx, MI_E_ARG, "matmul: op(A) is [%lld, %lld], op(B) is [%lld, %lld]", (long long)p.M, (long long)p.K,
                  (long long)kb, (long long)p.N);
    p.batch = 1; p.sa = p.sb = p.sc = 0;
    p.lda = A->cols; p.ldb = B->cols;
  } else if (mode == 1) {
    if (batch < 1 || m < 0 || k < 0 || n < 0) return fail(ctx, MI_E_ARG, "batched matmul dims");
    p.M = m; p.K = k; p.N = n; p.batch = batch;
    const int64_t a_item = m * k, b_item = k * n;
    const int64_t a_rows = ta ? k : m, a_cols = ta ? m : k;
    const int64_t b_rows = tb ? n : k, b_cols = tb ? k : n;
    if (A->cols != a_cols || (A->rows != a_rows && A->rows != a_rows * batch))
      return fail(ctx, MI_E_ARG, "batched matmul: A is [%lld, %lld], items [%lld, %lld] x %lld", (long long)A->rows,
                  (long long)A->cols, (long long)a_rows, (long long)a_cols, (long long)batch);
    if (B->cols != b_cols || (B->rows != b_rows && B->rows != b_rows * batch))
      return fail(ctx, MI_E_ARG, "batched matmul: B is [%lld, %lld], items [%lld, %lld] x %lld", (long long)B->rows,
                  (long long)B->cols, (long long)b_rows, (long long)b_cols, (long long)batch);
    p.sa = (A->rows == a_rows && batch > 1) ? 0 : a_item;
    p.sb = (B->rows == b_rows && batch > 1) ? 0 : b_item;
    p.sc = m * n;
    p.lda = a_cols; p.ldb = b_cols;
  } else {
    if (batch < 1 || m < 0 || k < 0 || n < 0 || !blk) return fail(ctx, MI_E_ARG, "block matmul dims");
    p.M = m; p.K = k; p.N = n; p.batch = batch;
    const int64_t a_rows = ta ? k : m, a_cols = ta ? m : k;
    const int64_t b_rows = tb ? n : k, b_cols = tb ? k : n;
    p.lda = A->cols; p.ldb = B->cols;
    if (!items_in(A, batch, a_rows, a_cols, blk[0], blk[1], p.lda))
      return fail(ctx, MI_E_ARG, "block matmul: A items [%lld, %lld] at %lld + i * %lld exceed [%lld, %lld]",
                  (long long)a_rows, (long long)a_cols, (long long)blk[0], (long long)blk[1], (long long)A->rows,
                  (long long)A->cols);
    if (!items_in(B, batch, b_rows, b_cols, blk[2], blk[3], p.ldb))
      return fail(ctx, MI_E_ARG, "block matmul: B items [%lld, %lld] at %lld + i * %lld exceed [%lld, %lld]",
                  (long long)b_rows, (long long)b_cols, (long long)blk[2], (long long)blk[3], (long long)B->rows,
                  (long long)B->cols);
    const size_t ea = elem_size(A->elem), eb = elem_size(B->elem);
    p.a = static_cast<const char *>(A->ptr) + blk[0] * ea;
    p.b = static_cast<const char *>(B->ptr) + blk[2] * eb;
    p.sa = blk[1]; p.sb = blk[3]; p.sc = m * n;
  }
  if (p.batch > 65535) return fail(ctx, MI_E_ARG, "batched matmul: batch %lld above 65535", (long long)p.batch);
  p.bias = lin.bias; p.resid = lin.resid; p.ldr = lin.ldr;
  p.norm_gamma = lin.norm_gamma; p.norm_eps = lin.norm_eps; p.norm_out = lin.norm_out; p.norm_elem = lin.norm_elem;
  p.norm_done = lin.norm_done;
  mi_id id; Buffer *cb;
  int s = new_buffer(ctx, p.batch * p.M, p.N, out_elem, &id, &cb);
  if (s) return s;
  p.c = cb->ptr;
  if (p.M > 0 && p.N > 0) {
    hipError_t e = hipSuccess;
    if (p.K == 0 && (p.bias || p.resid)) {
      // Empty sums: the epilogue alone, through a one-slice reduce of zeros.
      float *zeros = static_cast<float *>(scratch(ctx, static_cast<size_t>(p.M * p.N) * sizeof(float)));
      if (!zeros) { mi_free(ctx, id); return fail(ctx, MI_E_OOM, "linear scratch"); }
      if (fill_zero(ctx, zeros, static_cast<size_t>(p.M * p.N) * sizeof(float))) e = hipErrorLaunchFailure;
      const unsigned g = static_cast<unsigned>((p.M * p.N + 255) / 256);
      if (e == hipSuccess && out_elem == MI_BF16)
        splitk_reduce<uint16_t><<<g, 256, 0, ctx->stream>>>(zeros, 1, p.M * p.N, p.N, static_cast<uint16_t *>(cb->ptr),
                                                             p.N, p.bias, p.resid, p.ldr);
      else if (e == hipSuccess)
        splitk_reduce<float><<<g, 256, 0, ctx->stream>>>(zeros, 1, p.M * p.N, p.N, static_cast<float *>(cb->ptr), p.N,
                                                          p.bias, p.resid, p.ldr);
      if (e == hipSuccess) e = hipGetLastError();
    } else if (p.K == 0) {
      if (fill_zero(ctx, cb->ptr, p.batch * p.M * p.N * elem_size(out_elem))) e = hipErrorLaunchFailure;
    } else {
      s = run_product(ctx, p);
      if (s) { mi_free(ctx, id); return s; }
    }
    if (e != hipSuccess) {
      mi_free(ctx, id);
      return fail(ctx, MI_E_HIP, "matmul launch: %s", hipGetErrorString(e));
    }
    s = check_launch(ctx, "matmul");
    if (s) { mi_free(ctx, id); return s; }
  }
  *out = id;
  return MI_OK;
}

// A BFP8 operand of a product is decoded to BF16 first (exact), so the
// product is the BF16 product of the same values; *tmp receives the decoded
// buffer's id (0 when `id` is not BFP8), for the caller to free.  The decode
// step's projections read BFP8 weights themselves (mi_norm_matvec,
// mi_norm_qkv_rope, mi_norm_qkv_attention).
static int bfp8_operand(mi_ctx *ctx, mi_id id, mi_id *tmp) {
  *tmp = 0;
  Buffer *b = lookup(ctx, id);
  if (!b || b->elem != MI_BFP8) return MI_OK;  // an unknown id is reported by the product
  return bfp8_decode_to(ctx, b, MI_BF16, tmp, nullptr);
}

extern "C" int mi_matmul(mi_ctx *ctx, mi_id a, int a_transposed, mi_id b, int b_transposed, int out_elem, mi_id *out) {
  MI_ENTER(ctx);
  mi_id da, db;
  if (int s = bfp8_operand(ctx, a, &da)) return s;
  if (int s = bfp8_operand(ctx, b, &db)) {
    if (da) mi_free(ctx, da);
    return s;
  }
  const int s = matmul_common(ctx, da ? da : a, a_transposed, db ? db : b, b_transposed, 1, 0, 0, 0, 0, nullptr,
                              out_elem, out);
  if (da) mi_free(ctx, da);
  if (db) mi_free(ctx, db);
  return s;
}

extern "C" int mi_matmul_slices(mi_ctx *ctx, mi_id a, int a_transposed, mi_id b, int b_transposed, mi_id *out,
                                int64_t *slices) {
  MI_ENTER(ctx);
  if (!out || !slices) return fail(ctx, MI_E_ARG, "null out pointer");
  MI_BUF(ctx, A, a);
  MI_BUF(ctx, B, b);
  if (!elem_float(A->elem) || !elem_float(B->elem))
    return fail(ctx, MI_E_ARG, "matmul_slices of %s and %s", elem_name(A->elem), elem_name(B->elem));
  Plan p;
  p.ta = a_transposed != 0; p.tb = b_transposed != 0;
  p.fast = ctx->matmul_mode == MI_MATMUL_FAST;
  p.ea = A->elem; p.eb = B->elem; p.eo = MI_F32;
  p.a = A->ptr; p.b = B->ptr;
  p.M = p.ta ? A->cols : A->rows;
  p.K = p.ta ? A->rows : A->cols;
  const int64_t kb = p.tb ? B->cols : B->rows;
  p.N = p.tb ? B->rows : B->cols;
  if (kb != p.K)
    return fail(ctx, MI_E_ARG, "matmul_slices: op(A) is [%lld, %lld], op(B) is [%lld, %lld]", (long long)p.M,
                (long long)p.K, (long long)kb, (long long)p.N);
  p.batch = 1; p.sa = p.sb = p.sc = 0;
  p.lda = A->cols; p.ldb = B->cols;
  p.splits = (p.M > 0 && p.N > 0 && p.K > 0 && !gemv_fits(p)) ? splitk_slices(p) : 1;
  if (p.splits <= 1) {
    *slices = 1;
    return matmul_common(ctx, a, a_transposed, b, b_transposed, 1, 0, 0, 0, 0, nullptr, MI_F32, out);
  }
  plan_slices(p);
  mi_id id; Buffer *cb;
  int s = new_buffer(ctx, p.splits * p.M, p.N, MI_F32, &id, &cb);
  if (s) return s;
  hipError_t e = run_slices(p, static_cast<float *>(cb->ptr), ctx->stream);
  if (e != hipSuccess) {
    mi_free(ctx, id);
    return fail(ctx, MI_E_HIP, "matmul_slices launch: %s", hipGetErrorString(e));
  }
  s = check_launch(ctx, "matmul_slices");
  if (s) { mi_free(ctx, id); return s; }
  *out = id;
  *slices = p.splits;
  return MI_OK;
}

// A linear layer's bias (n elements) and residual ([m, n]), F32, each 0 for none.
static int linear_terms(mi_ctx *ctx, mi_id bias, mi_id residual, int64_t m, int64_t n, LinearTerms *lin) {
  if (bias) {
    MI_BUF(ctx, Bb, bias);
    if (Bb->elem != MI_F32 || Bb->numel() != n)
      return fail(ctx, MI_E_ARG, "linear: bias is %s [%lld, %lld], want F32 with %lld elements", elem_name(Bb->elem),
                  (long long)Bb->rows, (long long)Bb->cols, (long long)n);
    lin->bias = static_cast<const float *>(Bb->ptr);
  }
  if (residual) {
    MI_BUF(ctx, R, residual);
    if (R->elem != MI_F32 || R->rows != m || R->cols != n)
      return fail(ctx, MI_E_ARG, "linear: residual is %s [%lld, %lld], want F32 [%lld, %lld]", elem_name(R->elem),
                  (long long)R->rows, (long long)R->cols, (long long)m, (long long)n);
    lin->resid = static_cast<const float *>(R->ptr);
    lin->ldr = n;
  }
  return MI_OK;
}

extern "C" int mi_linear(mi_ctx *ctx, mi_id x, mi_id w, int w_transposed, mi_id bias, mi_id residual, int out_elem,
                         mi_id *out) {
  MI_ENTER(ctx);
  MI_BUF(ctx, X, x);
  MI_BUF(ctx, W, w);
  const int64_t m = X->rows, n = w_transposed ? W->rows : W->cols;
  LinearTerms lin;
  int s = linear_terms(ctx, bias, residual, m, n, &lin);
  if (s) return s;
  if (W->tiles) {
    if (!out) return fail(ctx, MI_E_ARG, "null out pointer");
    if (!w_transposed) return fail(ctx, MI_E_ARG, "linear: a weight in tiles is [n, k] (w_transposed 1)");
    return tiles_linear(ctx, x, w, lin.bias, lin.resid, out_elem, out);
  }
  mi_id dw;
  if ((s = bfp8_operand(ctx, w, &dw))) return s;
  s = matmul_common(ctx, x, 0, dw ? dw : w, w_transposed, 1, 0, 0, 0, 0, nullptr, out_elem, out, lin);
  if (dw) mi_free(ctx, dw);
  return s;
}

extern "C" int mi_linear_add_rms_norm(mi_ctx *ctx, mi_id x, mi_id w, int w_transposed, mi_id bias, mi_id residual,
                                      mi_id gamma, float eps, int norm_elem, mi_id *y, mi_id *y_norm) {
  MI_ENTER(ctx);
  if (!y || !y_norm) return fail(ctx, MI_E_ARG, "null out pointer");
  MI_BUF(ctx, X, x);
  MI_BUF(ctx, W, w);
  if (norm_elem != MI_F32 && norm_elem != MI_BF16 && norm_elem != MI_BF16_PARTS && norm_elem != MI_TILES_BF16 &&
      norm_elem != MI_TILES_PARTS)
    return fail(ctx, MI_E_ARG, "linear_add_rms_norm: norm result kind %d", norm_elem);
  const int64_t m = X->rows, n = w_transposed ? W->rows : W->cols;
  const float *gp = nullptr;
  if (gamma) {
    MI_BUF(ctx, G, gamma);
    if (G->elem != MI_F32 || G->numel() != n)
      return fail(ctx, MI_E_ARG, "linear_add_rms_norm: gain is %s [%lld, %lld], want F32 with %lld elements",
                  elem_name(G->elem), (long long)G->rows, (long long)G->cols, (long long)n);
    gp = static_cast<const float *>(G->ptr);
  }
  if (n > 8192) return fail(ctx, MI_E_UNSUPPORTED, "linear_add_rms_norm: rows of %lld (at most 8192)", (long long)n);
  LinearTerms lin;
  int s = linear_terms(ctx, bias, residual, m, n, &lin);
  if (s) return s;
  const bool tiled = norm_elem == MI_TILES_BF16 || norm_elem == MI_TILES_PARTS;
  const bool parts = norm_elem == MI_BF16_PARTS || norm_elem == MI_TILES_PARTS;
  if (tiled && (m % 32 || n % 16))
    return fail(ctx, MI_E_ARG, "linear_add_rms_norm: tiles of [%lld, %lld] (rows a multiple of 32, columns of 16)",
                (long long)m, (long long)n);
  if (W->tiles && !w_transposed)
    return fail(ctx, MI_E_ARG, "linear_add_rms_norm: a weight in tiles is [n, k] (w_transposed 1)");
  mi_id nid;
  Buffer *nb;
  if ((s = new_buffer(ctx, m, parts ? 2 * n : n, parts || tiled ? MI_BF16 : norm_elem, &nid, &nb))) return s;
  nb->tiles = tiled ? norm_elem : 0;
  bool done = false;
  if (!tiled) {  // the split-K reduce forms the row-major forms
    lin.norm_gamma = gp;
    lin.norm_eps = eps;
    lin.norm_out = nb->ptr;
    lin.norm_elem = norm_elem;
    lin.norm_done = &done;
  }
  mi_id dw = 0, yid = 0;
  if (W->tiles) {
    s = tiles_linear(ctx, x, w, lin.bias, lin.resid, MI_F32, &yid);
  } else {
    if ((s = bfp8_operand(ctx, w, &dw))) {
      mi_free(ctx, nid);
      return s;
    }
    s = matmul_common(ctx, x, 0, dw ? dw : w, w_transposed, 1, 0, 0, 0, 0, nullptr, MI_F32, &yid, lin);
  }
  if (dw) mi_free(ctx, dw);
  if (s) {
    mi_free(ctx, nid);
    return s;
  }
  if (!done && m > 0 && n > 0) {  // the product did not split over k: the norm's own launch
    rms_norm_launch(ctx, lookup(ctx, yid)->ptr, MI_F32, gp, MI_F32, eps, nb->ptr, norm_elem, m, n);
    if ((s = check_launch(ctx, "linear_add_rms_norm"))) {
      mi_free(ctx, yid);
      mi_free(ctx, nid);
      return s;
    }
  }
  *y = yid;
  *y_norm = nid;
  return MI_OK;
}

extern "C" int mi_linear_parts(mi_ctx *ctx, mi_id x_parts, mi_id w, int w_transposed, mi_id bias, mi_id residual,
                               int out_elem, mi_id *out) {
  MI_ENTER(ctx);
  if (!out) return fail(ctx, MI_E_ARG, "null out pointer");
  MI_BUF(ctx, X, x_parts);
  MI_BUF(ctx, W, w);
  if (X->elem != MI_BF16 || X->cols % 2 || X->tiles || W->tiles)
    return fail(ctx, MI_E_ARG, "linear_parts: parts are %s [%lld, %lld]%s, want BF16 [m, 2 k] rows (tiles go to mi_linear)",
                elem_name(X->elem), (long long)X->rows, (long long)X->cols, X->tiles || W->tiles ? " in tiles" : "");
  if (W->elem != MI_BF16) return fail(ctx, MI_E_ARG, "linear_parts: weight is %s, want BF16", elem_name(W->elem));
  if (out_elem != MI_F32 && out_elem != MI_BF16)
    return fail(ctx, MI_E_ARG, "linear_parts result kind %s", elem_name(out_elem));
  const int64_t m = X->rows, k = X->cols / 2, wk = w_transposed ? W->cols : W->rows, n = w_transposed ? W->rows : W->cols;
  if (wk != k)
    return fail(ctx, MI_E_ARG, "linear_parts: x is [%lld, %lld] (parts [%lld, %lld]), op(w) is [%lld, %lld]",
                (long long)m, (long long)k, (long long)m, (long long)(2 * k), (long long)wk, (long long)n);
  LinearTerms lin;
  int s = linear_terms(ctx, bias, residual, m, n, &lin);
  if (s) return s;
  Plan p;
  p.ta = false; p.tb = w_transposed != 0;
  p.fast = true;
  p.ea = MI_F32; p.eb = MI_BF16; p.eo = out_elem;
  p.a = nullptr; p.b = W->ptr;
  p.M = m; p.K = k; p.N = n;
  p.batch = 1; p.sa = p.sb = p.sc = 0;
  p.lda = k; p.ldb = W->cols;
  p.bias = lin.bias; p.resid = lin.resid; p.ldr = lin.ldr;
  if (k == 0 || !parts_direct_fits(p)) {
    // Any other shape: the weight repeated along k ([w | w] rows, or w over
    // w), then the plain BF16 product over 2 k -- the same sums.
    mi_id did; Buffer *db;
    s = new_buffer(ctx, p.tb ? n : 2 * k, p.tb ? 2 * k : n, MI_BF16, &did, &db);
    if (s) return s;
    hipError_t e = hipSuccess;
    for (int h = 0; h < 2 && e == hipSuccess && n > 0 && k > 0; ++h) {
      if (p.tb)
        e = hipMemcpy2DAsync(static_cast<uint16_t *>(db->ptr) + h * k, 2 * k * sizeof(uint16_t), W->ptr,
                             k * sizeof(uint16_t), k * sizeof(uint16_t), n, hipMemcpyDeviceToDevice, ctx->stream);
      else
        e = hipMemcpyAsync(static_cast<uint16_t *>(db->ptr) + h * k * n, W->ptr, k * n * sizeof(uint16_t),
                           hipMemcpyDeviceToDevice, ctx->stream);
    }
    if (e != hipSuccess) {
      mi_free(ctx, did);
      return fail(ctx, MI_E_HIP, "linear_parts copy: %s", hipGetErrorString(e));
    }
    s = matmul_common(ctx, x_parts, 0, did, w_transposed, 1, 0, 0, 0, 0, nullptr, out_elem, out, lin);
    mi_free(ctx, did);  // stream-ordered
    return s;
  }
  mi_id id; Buffer *cb;
  s = new_buffer(ctx, m, n, out_elem, &id, &cb);
  if (s) return s;
  p.c = cb->ptr;
  hipError_t e = hipSuccess;
  if (m > 0 && n > 0) e = launch_parts(p, X->ptr, ctx->stream);
  if (e != hipSuccess) {
    mi_free(ctx, id);
    return fail(ctx, MI_E_HIP, "linear_parts launch: %s", hipGetErrorString(e));
  }
  s = check_launch(ctx, "linear_parts");
  if (s) { mi_free(ctx, id); return s; }
  *out = id;
  return MI_OK;
}

extern "C" int mi_linear_swiglu_parts(mi_ctx *ctx, mi_id x_parts, mi_id w_pairs, mi_id *out) {
  MI_ENTER(ctx);
  if (!out) return fail(ctx, MI_E_ARG, "null out pointer");
  MI_BUF(ctx, X, x_parts);
  MI_BUF(ctx, W, w_pairs);
  if (X->elem != MI_BF16 || X->cols % 2 || W->elem != MI_BF16 || X->tiles || W->tiles)
    return fail(ctx, MI_E_ARG, "linear_swiglu_parts: parts %s [%lld, %lld] and weight %s, want BF16 [m, 2 k] and BF16 rows",
                elem_name(X->elem), (long long)X->rows, (long long)X->cols, elem_name(W->elem));
  const int64_t m = X->rows, k = X->cols / 2, n = W->rows;
  if (W->cols != k)
    return fail(ctx, MI_E_ARG, "linear_swiglu_parts: x is [%lld, %lld], the weight [%lld, %lld]", (long long)m,
                (long long)k, (long long)n, (long long)W->cols);
  Plan p;
  p.ta = false; p.tb = true;
  p.fast = true;
  p.ea = MI_F32; p.eb = MI_BF16; p.eo = MI_F32;
  p.a = nullptr; p.b = W->ptr;
  p.M = m; p.K = k; p.N = n;
  p.batch = 1; p.sa = p.sb = p.sc = 0;
  p.lda = k; p.ldb = W->cols;
  p.swiglu = SWIGLU_PARTS;
  // Whole tiles only (the pairs' epilogue has no edge form): 128-row tiles,
  // k a multiple of 32, 256 weight rows (128 outputs) a tile column.
  if (m < 1 || k < 1 || n % 256 || !parts_direct_fits(p))
    return fail(ctx, MI_E_UNSUPPORTED, "linear_swiglu_parts: [%lld, %lld] x [%lld, %lld] (m a multiple of 128, k of 32, "
                "the weight's rows of 256)", (long long)m, (long long)k, (long long)n, (long long)k);
  mi_id id; Buffer *cb;
  int s = new_buffer(ctx, m, n, MI_BF16, &id, &cb);
  if (s) return s;
  p.c = cb->ptr;
  const hipError_t e = launch_parts(p, X->ptr, ctx->stream);
  if (e != hipSuccess) {
    mi_free(ctx, id);
    return fail(ctx, MI_E_HIP, "linear_swiglu_parts launch: %s", hipGetErrorString(e));
  }
  s = check_launch(ctx, "linear_swiglu_parts");
  if (s) { mi_free(ctx, id); return s; }
  *out = id;
  return MI_OK;
}

extern "C" int mi_linear_swiglu(mi_ctx *ctx, mi_id x, mi_id w_pairs, int out_elem, mi_id *out) {
  MI_ENTER(ctx);
  if (!out) return fail(ctx, MI_E_ARG, "null out pointer");
  MI_BUF(ctx, X, x);
  MI_BUF(ctx, W, w_pairs);
  if (W->tiles) return tiles_swiglu(ctx, x, w_pairs, out_elem, out);
  if (X->elem != MI_BF16 || W->elem != MI_BF16 || X->tiles)
    return fail(ctx, MI_E_ARG, "linear_swiglu: x %s and weight %s, want BF16", elem_name(X->elem), elem_name(W->elem));
  if (out_elem != MI_F32 && out_elem != MI_BF16)
    return fail(ctx, MI_E_ARG, "linear_swiglu result kind %d", out_elem);
  const int64_t m = X->rows, k = X->cols, n = W->rows;
  if (W->cols != k)
    return fail(ctx, MI_E_ARG, "linear_swiglu: x is [%lld, %lld], the weight [%lld, %lld]", (long long)m, (long long)k,
                (long long)n, (long long)W->cols);
  Plan p;
  p.ta = false; p.tb = true;
  p.fast = true;
  p.ea = MI_BF16; p.eb = MI_BF16; p.eo = MI_F32;
  p.a = X->ptr; p.b = W->ptr;
  p.M = m; p.K = k; p.N = n;
  p.batch = 1; p.sa = p.sb = p.sc = 0;
  p.lda = k; p.ldb = W->cols;
  p.swiglu = out_elem == MI_BF16 ? SWIGLU_BF16 : SWIGLU_F32;
  if (m < 1 || k < 1 || n % 256 || !parts_direct_fits(p) || k % 8 || (reinterpret_cast<uintptr_t>(p.a) & 15))
    return fail(ctx, MI_E_UNSUPPORTED, "linear_swiglu: [%lld, %lld] x [%lld, %lld] (m a multiple of 128, k of 32, "
                "the weight's rows of 256)", (long long)m, (long long)k, (long long)n, (long long)k);
  mi_id id; Buffer *cb;
  int s = new_buffer(ctx, m, n / 2, out_elem, &id, &cb);
  if (s) return s;
  p.c = cb->ptr;
  hipError_t e;
  if (parts_small_tiles(p)) e = launch_pipe<float, 128, 128, 5, 2, 2>(p, ctx->stream);
  else e = launch_pipe<float, 256, 256, 5, 2, 4>(p, ctx->stream);
  if (e != hipSuccess) {
    mi_free(ctx, id);
    return fail(ctx, MI_E_HIP, "linear_swiglu launch: %s", hipGetErrorString(e));
  }
  s = check_launch(ctx, "linear_swiglu");
  if (s) { mi_free(ctx, id); return s; }
  *out = id;
  return MI_OK;
}

// mi_linear_qkv_rope_cache against a weight in tiles: the same checks of
// the tables and caches, then the short-row kernel with the tail.
static int linear_qkv_tiles(mi_ctx *ctx, const Buffer *X, const Buffer *W, const Buffer *cb, const Buffer *sb, int64_t seq,
                            int64_t heads, int64_t kv_heads, int64_t pos0, const Buffer *kb, const Buffer *vb,
                            int grouped, mi_id x, mi_id w_qkv, mi_id *q_out) {
  if (cb->elem != MI_F32 || sb->elem != MI_F32 || kb->elem != vb->elem || !elem_float(kb->elem))
    return fail(ctx, MI_E_ARG, "linear_qkv_rope_cache takes F32 tables and two F32 or two BF16 caches");
  const int64_t R = X->rows, D = kb->cols;
  if (heads < 1 || kv_heads < 1 || heads % kv_heads)
    return fail(ctx, MI_E_ARG, "linear_qkv_rope_cache: %lld heads over %lld kv heads", (long long)heads,
                (long long)kv_heads);
  if (D != 64)
    return fail(ctx, MI_E_UNSUPPORTED, "linear_qkv_rope_cache: head width %lld (64-wide heads)", (long long)D);
  if (W->rows != (heads + 2 * kv_heads) * D)
    return fail(ctx, MI_E_ARG, "linear_qkv_rope_cache: weight [%lld, %lld], want [(heads + 2 kv_heads) %lld, k]",
                (long long)W->rows, (long long)W->cols, (long long)D);
  if (seq < 1 || R % seq)
    return fail(ctx, MI_E_ARG, "linear_qkv_rope_cache: %lld rows are not sequences of %lld", (long long)R, (long long)seq);
  const int64_t batch = R / seq;
  if (vb->cols != D || vb->rows != kb->rows || kb->rows % (batch * kv_heads))
    return fail(ctx, MI_E_ARG, "linear_qkv_rope_cache: caches must both be [%lld * %lld * max_ctx, %lld]",
                (long long)batch, (long long)kv_heads, (long long)D);
  const int64_t maxc = kb->rows / (batch * kv_heads);
  if (pos0 < 0 || pos0 + seq > maxc)
    return fail(ctx, MI_E_ARG, "linear_qkv_rope_cache: positions [%lld, %lld) beyond the cache's %lld", (long long)pos0,
                (long long)(pos0 + seq), (long long)maxc);
  if (cb->cols != D || sb->cols != D || cb->rows != sb->rows || pos0 + seq > cb->rows)
    return fail(ctx, MI_E_ARG, "linear_qkv_rope_cache: rope tables [%lld, %lld] for positions below %lld",
                (long long)cb->rows, (long long)cb->cols, (long long)(pos0 + seq));
  mi_id id;
  Buffer *ob;
  if (int s = new_buffer(ctx, R * heads, D, MI_F32, &id, &ob)) return s;
  QkvTail t;
  t.mode = kb->elem == MI_BF16 ? QKV_BF16 : QKV_F32;
  t.cos = static_cast<const float *>(cb->ptr);
  t.sin = static_cast<const float *>(sb->ptr);
  t.q = static_cast<float *>(ob->ptr);
  t.kc = kb->ptr;
  t.vc = vb->ptr;
  t.seq = seq; t.pos0 = pos0; t.maxc = maxc;
  t.heads = static_cast<int>(heads); t.kvh = static_cast<int>(kv_heads); t.grouped = grouped != 0;
  if (int s = tiles_qkv(ctx, x, w_qkv, t)) {
    mi_free(ctx, id);
    return s;
  }
  *q_out = id;
  return MI_OK;
}

extern "C" int mi_linear_qkv_rope_cache(mi_ctx *ctx, mi_id x, int x_parts, mi_id w_qkv, mi_id cos_table,
                                        mi_id sin_table, int64_t seq, int64_t heads, int64_t kv_heads, int64_t pos0,
                                        mi_id k_cache, mi_id v_cache, int grouped, mi_id *q_out) {
  MI_ENTER(ctx);
  if (!q_out) return fail(ctx, MI_E_ARG, "null out pointer");
  MI_BUF(ctx, X, x);
  MI_BUF(ctx, W, w_qkv);
  MI_BUF(ctx, cb, cos_table);
  MI_BUF(ctx, sb, sin_table);
  MI_BUF(ctx, kb, k_cache);
  MI_BUF(ctx, vb, v_cache);
  if (W->tiles) return linear_qkv_tiles(ctx, X, W, cb, sb, seq, heads, kv_heads, pos0, kb, vb, grouped, x, w_qkv, q_out);
  if (X->elem != MI_BF16 || W->elem != MI_BF16 || (x_parts && X->cols % 2) || X->tiles)
    return fail(ctx, MI_E_ARG, "linear_qkv_rope_cache: x %s [%lld, %lld] (%s) and weight %s, want BF16",
                elem_name(X->elem), (long long)X->rows, (long long)X->cols, x_parts ? "parts" : "values",
                elem_name(W->elem));
  if (cb->elem != MI_F32 || sb->elem != MI_F32 || kb->elem != vb->elem || !elem_float(kb->elem))
    return fail(ctx, MI_E_ARG, "linear_qkv_rope_cache takes F32 tables and two F32 or two BF16 caches");
  const int64_t R = X->rows, K = x_parts ? X->cols / 2 : X->cols, D = kb->cols;
  if (heads < 1 || kv_heads < 1 || heads % kv_heads)
    return fail(ctx, MI_E_ARG, "linear_qkv_rope_cache: %lld heads over %lld kv heads", (long long)heads,
                (long long)kv_heads);
  const int64_t N = (heads + 2 * kv_heads) * D;
  if (W->rows != N || W->cols != K)
    return fail(ctx, MI_E_ARG, "linear_qkv_rope_cache: weight [%lld, %lld], want [(heads + 2 kv_heads) %lld, %lld]",
                (long long)W->rows, (long long)W->cols, (long long)D, (long long)K);
  if (seq < 1 || R % seq)
    return fail(ctx, MI_E_ARG, "linear_qkv_rope_cache: %lld rows are not sequences of %lld", (long long)R, (long long)seq);
  const int64_t batch = R / seq;
  if (vb->cols != D || vb->rows != kb->rows || kb->rows % (batch * kv_heads))
    return fail(ctx, MI_E_ARG, "linear_qkv_rope_cache: caches must both be [%lld * %lld * max_ctx, %lld]",
                (long long)batch, (long long)kv_heads, (long long)D);
  const int64_t maxc = kb->rows / (batch * kv_heads);
  if (pos0 < 0 || pos0 + seq > maxc)
    return fail(ctx, MI_E_ARG, "linear_qkv_rope_cache: positions [%lld, %lld) beyond the cache's %lld", (long long)pos0,
                (long long)(pos0 + seq), (long long)maxc);
  if (cb->cols != D || sb->cols != D || cb->rows != sb->rows || pos0 + seq > cb->rows)
    return fail(ctx, MI_E_ARG, "linear_qkv_rope_cache: rope tables [%lld, %lld] for positions below %lld",
                (long long)cb->rows, (long long)cb->cols, (long long)(pos0 + seq));
  Plan p;
  p.ta = false; p.tb = true;
  p.fast = true;
  p.ea = x_parts ? MI_F32 : MI_BF16; p.eb = MI_BF16; p.eo = MI_F32;
  p.a = X->ptr; p.b = W->ptr; p.c = nullptr;
  p.M = R; p.K = K; p.N = N;
  p.batch = 1; p.sa = p.sb = p.sc = 0;
  p.lda = X->cols; p.ldb = W->cols;
  if (D != 64 || R < 1 || !parts_direct_fits(p) || (reinterpret_cast<uintptr_t>(X->ptr) & 15))
    return fail(ctx, MI_E_UNSUPPORTED, "linear_qkv_rope_cache: [%lld, %lld] x [%lld, %lld], head width %lld (64-wide "
                "heads, rows a multiple of 128, k of 32)", (long long)R, (long long)K, (long long)N, (long long)K,
                (long long)D);
  mi_id id; Buffer *ob;
  int s = new_buffer(ctx, R * heads, D, MI_F32, &id, &ob);
  if (s) return s;
  p.qkv.mode = kb->elem == MI_BF16 ? QKV_BF16 : QKV_F32;
  p.qkv.cos = static_cast<const float *>(cb->ptr);
  p.qkv.sin = static_cast<const float *>(sb->ptr);
  p.qkv.q = static_cast<float *>(ob->ptr);
  p.qkv.kc = kb->ptr;
  p.qkv.vc = vb->ptr;
  p.qkv.seq = seq; p.qkv.pos0 = pos0; p.qkv.maxc = maxc;
  p.qkv.heads = static_cast<int>(heads); p.qkv.kvh = static_cast<int>(kv_heads); p.qkv.grouped = grouped != 0;
  const hipError_t e = x_parts ? launch_parts(p, X->ptr, ctx->stream) : launch_direct(p, ctx->stream);
  if (e != hipSuccess) {
    mi_free(ctx, id);
    return fail(ctx, MI_E_HIP, "linear_qkv_rope_cache launch: %s", hipGetErrorString(e));
  }
  s = check_launch(ctx, "linear_qkv_rope_cache");
  if (s) { mi_free(ctx, id); return s; }
  *q_out = id;
  return MI_OK;
}

extern "C" int mi_matmul_items(mi_ctx *ctx, mi_id a, int a_transposed, const int64_t *a_at, mi_id b,
                               int b_transposed, const int64_t *b_at, int64_t groups, int64_t per_group, int64_t m,
                               int64_t k, int64_t n, mi_id out, const int64_t *out_at) {
  MI_ENTER(ctx);
  if (!a_at || !b_at || !out_at) return fail(ctx, MI_E_ARG, "null item placement");
  MI_BUF(ctx, A, a);
  MI_BUF(ctx, B, b);
  MI_BUF(ctx, C, out);
  if (out == a || out == b) return fail(ctx, MI_E_ARG, "matmul_items: the result buffer is also an operand");
  if (!elem_float(A->elem) || !elem_float(B->elem) || !elem_float(C->elem))
    return fail(ctx, MI_E_ARG, "matmul_items of %s and %s into %s", elem_name(A->elem), elem_name(B->elem),
                elem_name(C->elem));
  if (groups < 1 || per_group < 1 || m < 1 || k < 1 || n < 1)
    return fail(ctx, MI_E_ARG, "matmul_items: %lld x %lld items of [%lld, %lld] x [%lld, %lld]", (long long)groups,
                (long long)per_group, (long long)m, (long long)k, (long long)k, (long long)n);
  if (groups > 65535 || per_group > 65535 || groups * per_group > 65535)
    return fail(ctx, MI_E_ARG, "matmul_items: %lld x %lld items, above 65535", (long long)groups,
                (long long)per_group);
  const int ta = a_transposed != 0, tb = b_transposed != 0;
  const int64_t a_rows = ta ? k : m, a_cols = ta ? m : k;
  const int64_t b_rows = tb ? n : k, b_cols = tb ? k : n;
  if (!grouped_items_in(A, groups, per_group, a_rows, a_cols, a_at))
    return fail(ctx, MI_E_ARG, "matmul_items: A items [%lld, %lld] at %lld + g * %lld + i * %lld exceed [%lld, %lld]",
                (long long)a_rows, (long long)a_cols, (long long)a_at[0], (long long)a_at[1], (long long)a_at[2],
                (long long)A->rows, (long long)A->cols);
  if (!grouped_items_in(B, groups, per_group, b_rows, b_cols, b_at))
    return fail(ctx, MI_E_ARG, "matmul_items: B items [%lld, %lld] at %lld + g * %lld + i * %lld exceed [%lld, %lld]",
                (long long)b_rows, (long long)b_cols, (long long)b_at[0], (long long)b_at[1], (long long)b_at[2],
                (long long)B->rows, (long long)B->cols);
  if (!grouped_items_in(C, groups, per_group, m, n, out_at))
    return fail(ctx, MI_E_ARG,
                "matmul_items: result items [%lld, %lld] at %lld + g * %lld + i * %lld exceed [%lld, %lld]",
                (long long)m, (long long)n, (long long)out_at[0], (long long)out_at[1], (long long)out_at[2],
                (long long)C->rows, (long long)C->cols);
  Plan p;
  p.ta = ta; p.tb = tb;
  p.fast = ctx->matmul_mode == MI_MATMUL_FAST;
  p.ea = A->elem; p.eb = B->elem; p.eo = C->elem;
  p.M = m; p.K = k; p.N = n; p.batch = groups * per_group;
  p.a = static_cast<const char *>(A->ptr) + a_at[0] * elem_size(A->elem);
  p.b = static_cast<const char *>(B->ptr) + b_at[0] * elem_size(B->elem);
  p.c = static_cast<char *>(C->ptr) + out_at[0] * elem_size(C->elem);
  p.lda = A->cols; p.ldb = B->cols; p.ldc = C->cols;
  p.per_group = per_group;
  p.sa = a_at[2]; p.sb = b_at[2]; p.sc = out_at[2];
  p.sa2 = a_at[1]; p.sb2 = b_at[1]; p.sc2 = out_at[1];
  return run_product(ctx, p);
}

extern "C" int mi_set_matmul_mode(mi_ctx *ctx, int mode) {
  MI_ENTER(ctx);
  if (mode != MI_MATMUL_FAST && mode != MI_MATMUL_ACCURATE)
    return fail(ctx, MI_E_UNSUPPORTED, "matmul mode %d (fast %d, accurate %d)", mode, MI_MATMUL_FAST,
                MI_MATMUL_ACCURATE);
  ctx->matmul_mode = mode;
  return MI_OK;
}

extern "C" int mi_get_matmul_mode(mi_ctx *ctx, int *mode) {
  MI_ENTER(ctx);
  if (!mode) return fail(ctx, MI_E_ARG, "null out pointer");
  *mode = ctx->matmul_mode;
  return MI_OK;
}

extern "C" int mi_matmul_blocks(mi_ctx *ctx, mi_id a, int a_transposed, mi_id b, int b_transposed, int64_t batch,
                                int64_t m, int64_t k, int64_t n, int64_t a_offset, int64_t a_stride, int64_t b_offset,
                                int64_t b_stride, int out_elem, mi_id *out) {
  MI_ENTER(ctx);
  const int64_t blk[4] = {a_offset, a_stride, b_offset, b_stride};
  return matmul_common(ctx, a, a_transposed, b, b_transposed, batch, m, k, n, 2, blk, out_elem, out);
}

extern "C" int mi_matmul_batched(mi_ctx *ctx, mi_id a, int a_transposed, mi_id b, int b_transposed, int64_t batch,
                                 int64_t m, int64_t k, int64_t n, int out_elem, mi_id *out) {
  MI_ENTER(ctx);
  return matmul_common(ctx, a, a_transposed, b, b_transposed, batch, m, k, n, 1, nullptr, out_elem, out);
}
