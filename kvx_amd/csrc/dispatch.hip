// Host-side launch planning: picks a kernel family, its chunk width, tile
// shape and grid for a validated write or gather plan, and enqueues it on
// the caller's stream through the run_* entry points of kernels.h.
#include <hip/hip_runtime.h>

#include "kernels.h"
#include "kvx_internal.h"

namespace kvx {
namespace dev {
namespace {

GeomBytes to_bytes(const Geom &g, int esize) {
  GeomBytes r;
  r.s_block = g.s_block * esize;
  r.s_off = g.s_off * esize;
  r.s_head = g.s_head * esize;
  r.s_piece = g.s_piece * esize;
  r.s_inner = g.s_inner * esize;
  r.pack = g.pack;
  r.pad_ = 0;
  return r;
}

bool aligned(const void *p, int64_t b) {
  return ((uintptr_t)p % (uintptr_t)b) == 0;
}

// True when chunks of g elements (g*esize bytes each) stay inside one
// contiguous cache piece and every cache address they use is aligned.  A
// block of one token never steps by the offset stride, nor a cache of one
// head by the head stride (size-1 axes, whose strides can be anything, e.g.
// 1 for vLLM's [num_blocks, H, D, 1] value cache).
bool cache_chunk_ok(const Geom &g, const void *base, int esize, int head_dim,
                    int ge, int64_t block_size, int64_t heads) {
  const int64_t bytes = (int64_t)ge * esize;
  if (ge > 1 && g.s_inner != 1) return false;
  if (g.pack % ge != 0 || head_dim % ge != 0) return false;
  if (!aligned(base, bytes)) return false;
  const int64_t strides[4] = {g.s_block, block_size == 1 ? 0 : g.s_off, heads == 1 ? 0 : g.s_head,
                              g.s_piece};
  for (int64_t st : strides) {
    if ((st * esize) % bytes != 0) return false;
  }
  return true;
}

// Widest chunk (elements) that works for K, V and the io buffers.  The io
// side is contiguous with rows of H*D elements of io_size bytes.
int pick_chunk(const Geom &gk, const Geom &gv, const void *ck, const void *cv,
               int cache_size, const void *ik, const void *iv, int io_size,
               int head_dim, int max_chunk_bytes_cache, int64_t block_size, int64_t heads) {
  for (int ge = max_chunk_bytes_cache / cache_size; ge >= 1; ge /= 2) {
    if (!cache_chunk_ok(gk, ck, cache_size, head_dim, ge, block_size, heads)) continue;
    if (!cache_chunk_ok(gv, cv, cache_size, head_dim, ge, block_size, heads)) continue;
    const int64_t io_bytes = (int64_t)ge * io_size;
    if (!aligned(ik, io_bytes) || !aligned(iv, io_bytes)) continue;
    return ge;
  }
  return 1;
}

int lpt_log2_for(int nchunks) {
  int lg = 0;
  while ((1 << lg) < nchunks && lg < 6) ++lg;
  return lg;
}

hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

// HIP's limits on one grid dimension: at most 2^31 - 1 workgroups and
// 2^32 - 1 work-items (gridDim.x * blockDim.x).
bool grid_fits(int64_t workgroups, int threads) {
  return workgroups <= 0x7FFFFFFF && workgroups * threads <= 0xFFFFFFFFll;
}

int log2_exact(int64_t v) {
  if (v <= 0 || (v & (v - 1)) != 0) return -1;
  int lg = 0;
  while ((int64_t(1) << lg) < v) ++lg;
  return lg;
}

// Row (head, dim) elements at consecutive addresses: row-major layouts, and
// any dense layout whose block holds one row (HND, x-packed or token axis
// innermost with block_size 1 store a row as H * D consecutive elements).
// With one head the head stride is never used (HND with H = 1 is row-major
// whenever rows are D elements apart).  On MI355X (c2's lengths in
// one-token blocks) such gathers took 1592-1615 us per layer in the flat
// kernel against 3517-3551 us in the tile kernels.
bool row_elems_contiguous(const Geom &g, int64_t D, int64_t H) {
  return g.s_inner == 1 && (g.s_head == D || H == 1) && (g.pack == D || g.s_piece == g.pack);
}

// Elements of one per-token contiguous run when `g` is a dense block in
// (run, offset, within-run) order, element e of row o at
// (e / W) * bs * W + o * W + e % W, else -1: W = H * D (row-major), D (HND),
// x (x-packed) or 1 (token axis innermost).  Any block stride.
int64_t dense_run_elems(const Geom &g, int64_t bs, int64_t H, int64_t D) {
  // one row, or rows of one head D elements apart: row-major
  if (row_elems_contiguous(g, D, H) && (bs == 1 || g.s_off == H * D)) return H * D;
  const int64_t p = g.pack;
  const bool split = p < D;  // d = (d / p) * p + d % p with its own strides
  if (g.s_inner == 1 && (!split || g.s_piece == p)) {
    if (g.s_off == H * D && g.s_head == D) return H * D;
    if (g.s_off == D && g.s_head == bs * D) return D;
  }
  if (split && g.s_inner == 1 && g.s_off == p && g.s_piece == bs * p && g.s_head == bs * D)
    return p;
  if (g.s_off == 1 && g.s_inner == bs && (!split || g.s_piece == bs * p) && g.s_head == bs * D)
    return 1;
  return -1;
}

// Transposing-gather plan (gather_tiles_kernel) for a PACKED-table gather of
// dense blocks of which at least one is not row-major, or false.  On MI355X
// (c2 shapes, bf16) it beats the row kernel for every run length measured:
// token-innermost 2.45 -> 5.90 TB/s, x-packed 4.66 -> 5.88, HND (256-byte
// runs) 5.14 -> 5.87.  kTileBytes is the cache bytes per tensor of one
// tile (8 KiB measured best against 4 and 16 KiB); workgroups have about
// one thread per kTileBytesPerThread bytes of tile.
constexpr int64_t kTileBytes = 8192;
constexpr int64_t kTileBytesPerThread = 32;
// Narrowest tile width (cache bytes per row) the halving below goes to.
constexpr int64_t kTileMinWidth = 128;
// Tiles whose width is not a power of two: at most kOddTileBytes of cache
// bytes per tensor, at least kOddTileMin.
constexpr int64_t kOddTileBytes = 12288;
constexpr int64_t kOddTileMin = 4096;

int64_t gcd64(int64_t a, int64_t b) {
  while (b != 0) {
    const int64_t t = a % b;
    a = b;
    b = t;
  }
  return a;
}

// div_magic's multiplier for divisor d >= 2: ceil(2^32 / d).
uint32_t magic_for(int64_t d) { return (uint32_t)(((uint64_t(1) << 32) + (uint64_t)d - 1) / (uint64_t)d); }

// Tile width of whole runs (a multiple of `unit`) that divides the row, for
// rows or runs that are not a power of two, phase 2 dividing by chunks per
// row with a multiply-high (HND heads of 96 or 80 bf16 elements, three
// 256-byte heads): widths of whole 128-byte lines first, then the tile
// nearest `target` bytes, the wider on a tie, within kOddTileMin and
// max(target, kOddTileBytes); -1 if none.  On MI355X (c2's table, 4
// layers) such gathers took 5-8% less time than in gather_rows_kernel;
// widths that split output lines between two workgroups (320 or 192
// bytes) measured 7-12% slower than line-multiple ones (640 or 384 bytes),
// three 256-byte heads 20% slower in 4 KiB tiles than in 12 KiB ones, and
// HND 8 x 96 bf16 3% faster in 6 KiB tiles than in 12 KiB ones.
int64_t odd_tile_width(int64_t row, int64_t unit, int64_t bs, int64_t target) {
  if (row % unit != 0) return -1;
  const int64_t cap = target > kOddTileBytes ? target : kOddTileBytes;
  int64_t tw = -1, best = 0;
  for (int64_t k = row / unit; k >= 1; --k) {
    if ((row / unit) % k != 0) continue;
    const int64_t w = unit * k, bytes = w * bs;
    if (bytes < kOddTileMin || bytes > cap) continue;
    const int64_t dist = bytes > target ? bytes - target : target - bytes;
    const int64_t score = (w % 128 == 0 ? 0 : (int64_t)1 << 40) + dist;
    if (tw < 0 || score < best) {
      tw = w;
      best = score;
    }
  }
  return tw;
}

// gather_rows_kernel: cache row bytes per tensor of one workgroup's share
// of a block, at least (blocks of up to kRowsTileBytes stay whole).
constexpr int64_t kRowsTileBytes = 32768;

bool plan_tiles(const GatherPlan &p, int cs, int is, int src_chunk, TileArgs *t,
                int64_t *grid, uint32_t *lds_bytes) {
  const bool offsets = p.format == KVX_BLOCK_TABLE_KV_OFFSETS;
  const bool ragged = p.format == KVX_BLOCK_TABLE_RAGGED;
  if (ragged && p.block_size > kTileMaxRows) return false;  // a tile's row ids in LDS
  const int64_t bs = p.block_size;
  const int64_t H = p.heads;
  const int64_t D = p.head_dim;
  const int64_t row_cache = H * D * cs;
  const int bs_log2 = log2_exact(bs);
  if (bs_log2 < 0 || row_cache < 16) return false;
  const Geom *g[2] = {&p.gk, &p.gv};
  const void *src[2] = {p.src_k, p.src_v};
  void *dst[2] = {p.dst_k, p.dst_v};
  int run_log2[2];
  int64_t run_bytes[2] = {0, 0};
  bool transposed = false, odd_run = false;
  int64_t min_tw = 16;
  int64_t unit = 16;  // a tile width holds whole runs and 16-byte chunks
  for (int i = 0; i < 2; ++i) {
    const int64_t w = dense_run_elems(*g[i], bs, H, D);
    if (w < 0) return false;
    run_log2[i] = w == H * D ? -1 : log2_exact(w * cs);
    if (w != H * D) {
      run_bytes[i] = w * cs;
      if (run_log2[i] < 0) {
        // runs that are not a power of two: 16-byte pieces, one run each
        if (run_bytes[i] % 16 != 0) return false;
        run_log2[i] = kRunOdd;
        odd_run = true;
      }
      transposed = true;
      if (w * cs > min_tw) min_tw = w * cs;
      unit = unit / gcd64(unit, run_bytes[i]) * run_bytes[i];
    }
    // block addresses: base + index * pitch, all 16-byte aligned
    const uintptr_t base =
        offsets ? reinterpret_cast<uintptr_t>(p.pool[0]) | reinterpret_cast<uintptr_t>(p.pool[1]) |
                      (uintptr_t)p.bytes_per_block
                : reinterpret_cast<uintptr_t>(src[i]) | (uintptr_t)(g[i]->s_block * cs);
    if (base % 16 != 0) return false;
    const int dst_align = src_chunk / cs * is;  // output bytes per chunk
    if (reinterpret_cast<uintptr_t>(dst[i]) % dst_align != 0) return false;
  }
  if (!transposed) return false;  // row-major pairs: the flat kernels
  // RAGGED blocks of more rows than a wave has lanes load their row ids with
  // every thread and one more barrier: taken where a tensor's runs are
  // narrower than a 128-byte line (x-packed, token axis innermost), which
  // the row kernel reads piece by piece.  On MI355X (c2's lengths, RAGGED,
  // 128-token blocks, same-box A/B) x-packed K and V 2715 -> 1720 us,
  // vLLM's pair 5455 -> 2019 us; HND (256-byte runs) 1640 -> 1718 us, so HND
  // keeps the row kernel.
  if (ragged && bs > kWave) {
    int64_t narrow = -1;
    for (int i = 0; i < 2; ++i)
      if (run_bytes[i] > 0 && (narrow < 0 || run_bytes[i] < narrow)) narrow = run_bytes[i];
    if (narrow >= 128) return false;
  }
  if ((D * cs) % src_chunk != 0) return false;  // chunks never straddle heads
  // Tile width: a power of two that divides the row and holds whole runs.
  // A row that is not a power of two (6 or 12 heads, say) makes several
  // tiles of its largest power-of-two divisor, when that still fills a tile:
  // on MI355X (c2's table) HND gathers of 6 x 128 and 12 x 64 bf16 heads
  // measured 0.676 of peak in 8 KiB tiles against 0.63 in gather_rows_kernel,
  // 3 x 128 heads 0.587 in 4 KiB tiles against 0.623.
  int64_t tw = row_cache & -row_cache;
  if (odd_run || tw < min_tw ||
      ((row_cache & (row_cache - 1)) != 0 && tw * bs < kTileBytes)) {
    tw = odd_tile_width(row_cache, unit, bs, kTileBytes);
    if (tw < 0) return false;
  } else {
    // halve toward kTileBytes, but not below one 128-byte output line per
    // row (blocks of 128 or 256 tokens then take 16 or 32 KiB tiles): on
    // MI355X (c2's lengths, bf16 x-packed blocks of 128 / 256 tokens) 2315 /
    // 6752 -> 1789 / 1823 us per layer, where narrower rows split output
    // lines between workgroups.  (Runs of whole lines, HND, also gathered
    // faster in these tiles than in gather_rows_kernel at every block size
    // that fits: 16-128 tokens, 4-12% at c2's size.)
    while (tw * bs > kTileBytes && tw / 2 >= min_tw && tw / 2 >= kTileMinWidth) tw /= 2;
  }
  const int64_t pitch = tw + kTilePad;
  if (bs * pitch > 64 * 1024) return false;
  t->table = p.block_table;
  t->seq_lens = p.seq_lens;
  t->indptr = p.indptr;
  t->table_count = p.table_count;
  t->pool[0] = p.pool[0];
  t->pool[1] = p.pool[1];
  t->bytes_per_block = p.bytes_per_block;
  t->pool_blocks[0] = p.pool_blocks[0];
  t->pool_blocks[1] = p.pool_blocks[1];
  t->out_row_bytes = H * D * is;
  t->max_blocks_per_seq = p.max_blocks_per_seq;
  const int64_t by_len = ((int64_t)p.max_seq_len + bs - 1) / bs;
  // RAGGED rows do not use max_blocks_per_seq
  t->blocks_per_seq = (int32_t)(ragged || by_len < p.max_blocks_per_seq ? by_len
                                                                       : p.max_blocks_per_seq);
  t->tiles = (int32_t)(row_cache / tw);
  t->tw = (int32_t)tw;
  t->tw_log2 = log2_exact(tw);
  // phase 2 chunks per row; div_magic is exact for u * cpr <= 2^32, and
  // u * cpr < bs * tw * tw <= 2^16 * tw (bs * pitch <= 64 KiB below)
  t->cpr = (int32_t)(tw / src_chunk);
  t->cpr_magic = t->tw_log2 < 0 ? magic_for(t->cpr) : 0;
  t->pitch = (int32_t)pitch;
  // Workgroups of about one thread per kTileBytesPerThread bytes of
  // tile (64 to 256 threads): smaller tiles run in smaller workgroups, more
  // of them resident per CU, so that as many bytes are in flight as for the
  // 8 KiB tiles of wider rows.  On MI355X (c2's table, one KV head) 4 KiB
  // x-packed tiles took 198.8 us in 128-thread workgroups against 259.9 us
  // in 256-thread and 209.7 us in 64-thread ones; HND two-token blocks 1585
  // against 2058 us per layer.
  t->threads = kBlockThreads;
  while (t->threads > 64 && tw * bs < (int64_t)t->threads * kTileBytesPerThread)
    t->threads /= 2;
  t->max_seq_len = p.max_seq_len;
  t->num_blocks = p.num_blocks;
  t->head_dim = p.head_dim;
  t->row_elems = (int32_t)(H * D);
  t->bs_log2 = bs_log2;
  t->cache_es_log2 = log2_exact(cs);
  t->io_es_log2 = log2_exact(is);
  const ScaleRef sc[2] = {p.k_scale, p.v_scale};
  for (int i = 0; i < 2; ++i) {
    t->t[i].src = static_cast<const char *>(src[i]);
    t->t[i].dst = static_cast<char *>(dst[i]);
    t->t[i].s_block = g[i]->s_block * cs;
    t->t[i].sc = sc[i];
    t->t[i].run_log2 = run_log2[i];
    // stage_tile_odd divides region offsets (< 64 KiB) by the run: exact
    // for runs below 2^16 bytes
    t->t[i].run_bytes = (int32_t)run_bytes[i];
    t->t[i].run_magic = run_log2[i] == kRunOdd ? magic_for(run_bytes[i]) : 0;
    t->t[i].pad_ = 0;
  }
  *grid = (int64_t)p.seq_count * t->blocks_per_seq * t->tiles;
  *lds_bytes = (uint32_t)(bs * pitch);
  return grid_fits(*grid, t->threads);
}

// Tiled block write plan (write_tiles_kernel): at least bs tokens,
// power-of-two bs (<= one wave) and cache row bytes, dense blocks of which
// at least one is not row-major, 16-byte aligned block addresses, io rows
// aligned to the tile op's source chunk, and (quantizing) heads a whole
// number of 8-element chunks, so that every chunk has one scale.
// kWriteTileBytes: cache bytes per tensor of one tile of a copying write;
// kQuantTileBytes the same for the FP8 quantizing write (whose
// io rows are 2-4x its cache bytes).  On MI355X (c3 shapes, inputs not
// cache-resident) 8 KiB measured 1.5-3% faster than 16 KiB for copies, and
// 4-5% faster than 32 or 64 KiB; the quantizing write is 4-8% faster with
// 16 KiB; 4 KiB is 25-30% slower for both.  Tiles are 0-5% faster than
// staging whole blocks of K and V in one workgroup (x-packed / HND), 5x for
// the token-innermost value cache.
constexpr int64_t kWriteTileBytes = 8192;
constexpr int64_t kQuantTileBytes = 16384;
bool plan_write_tiles(const WritePlan &p, int cs, int is, WriteTileArgs *wt, int64_t *grid,
                      uint32_t *lds_bytes) {
  const int64_t bs = p.block_size;
  const int64_t H = p.heads;
  const int64_t D = p.head_dim;
  const int64_t row_cache = H * D * cs;
  const int bs_log2 = log2_exact(bs);
  if (bs_log2 < 0 || bs > kWave || p.num_tokens < bs) return false;
  if (row_cache < 16) return false;
  const int src_chunk = p.conv == kConvQuant ? 8 * is : 16;
  if (p.conv == kConvQuant && D % 8 != 0) return false;
  const Geom *g[2] = {&p.gk, &p.gv};
  const void *src[2] = {p.src_k, p.src_v};
  const void *dst[2] = {p.dst_k, p.dst_v};
  bool transposed = false, odd_run = false;
  int64_t min_tw = 16;
  int64_t unit = 16;  // a tile width holds whole runs and 16-byte chunks
  for (int i = 0; i < 2; ++i) {
    const int64_t w = dense_run_elems(*g[i], bs, H, D);
    if (w < 0) return false;
    wt->run_log2[i] = w == H * D ? -1 : log2_exact(w * cs);
    wt->run_bytes[i] = 0;
    wt->run_magic[i] = 0;
    if (w != H * D) {
      if (wt->run_log2[i] < 0) {
        // runs that are not a power of two: 16-byte pieces, one run each
        if ((w * cs) % 16 != 0) return false;
        wt->run_log2[i] = kRunOdd;
        wt->run_bytes[i] = (int32_t)(w * cs);
        // unstage_tile_odd divides region offsets (< 64 KiB) by the run
        wt->run_magic[i] = magic_for(w * cs);
        odd_run = true;
      }
      transposed = true;
      if (w * cs > min_tw) min_tw = w * cs;
      unit = unit / gcd64(unit, w * cs) * (w * cs);
    }
    if ((reinterpret_cast<uintptr_t>(dst[i]) | (uintptr_t)(g[i]->s_block * cs)) % 16 != 0)
      return false;
    if ((reinterpret_cast<uintptr_t>(src[i]) | (uintptr_t)(H * D * is)) % src_chunk != 0)
      return false;
  }
  if (!transposed) return false;
  const int64_t tile_bytes =
      p.conv == kConvQuant ? kQuantTileBytes : kWriteTileBytes;
  // as in plan_tiles: a power-of-two tile width that divides the row, and
  // a full copy tile for a row that is not a power of two (c3's size into
  // HND caches of 6 x 128 or 12 x 64 bf16 heads: 0.527 of peak against 0.43
  // per token); otherwise a tile of whole runs (odd_tile_width): at c3's
  // size, 3 heads of 128 measured 0.61 of peak against 0.11 per token for
  // an x-packed K, 0.58 against 0.055 for vLLM's K / V pair and 0.68 against
  // 0.50 for HND; HND 8 x 80 0.61 against 0.50, 8 x 96 0.60 against 0.57
  int64_t tw = row_cache & -row_cache;
  if (odd_run || tw < min_tw ||
      ((row_cache & (row_cache - 1)) != 0 && tw * bs < kWriteTileBytes)) {
    tw = odd_tile_width(row_cache, unit, bs, tile_bytes);
    if (tw < 0) return false;
  } else {
    while (tw * bs > tile_bytes && tw / 2 >= min_tw) tw /= 2;
  }
  const int64_t pitch = tw + kTilePad;
  if (bs * pitch > 64 * 1024) return false;
  wt->tiles = (int32_t)(row_cache / tw);
  wt->tw = (int32_t)tw;
  wt->tw_log2 = log2_exact(tw);
  // phase 1 chunks per row (Op::kDst cache bytes each: 16, or 8 FP8 bytes);
  // div_magic is exact since u * cpr < bs * tw * tw <= 2^16 * tw
  wt->cpr = (int32_t)(tw / (p.conv == kConvQuant ? 8 : 16));
  wt->cpr_magic = wt->tw_log2 < 0 ? magic_for(wt->cpr) : 0;
  wt->pitch = (int32_t)pitch;
  // about one thread per kTileBytesPerThread bytes of tile, as for
  // the gather: small tiles (one KV head) in smaller workgroups.  On MI355X
  // (c3's bytes in one-head rows) vLLM's pair 61.3 -> 53.4 us, x-packed K
  // and V 58.6 -> 53.1 us; c3's own 8 KiB tiles unchanged.
  wt->threads = kBlockThreads;
  while (wt->threads > 64 && tw * bs < (int64_t)wt->threads * kTileBytesPerThread)
    wt->threads /= 2;
  wt->bs_log2 = bs_log2;
  wt->cache_es_log2 = log2_exact(cs);
  wt->io_es_log2 = log2_exact(is);
  *grid = (p.num_tokens + bs - 1) / bs * wt->tiles;
  *lds_bytes = (uint32_t)(bs * pitch);
  return grid_fits(*grid, wt->threads);
}

}  // namespace
}  // namespace dev

using namespace dev;

int dtype_size(kvx_dtype_t dt) {
  switch (dt) {
    case KVX_DTYPE_F32: return 4;
    case KVX_DTYPE_F16:
    case KVX_DTYPE_BF16: return 2;
    case KVX_DTYPE_F8_E4M3:
    case KVX_DTYPE_F8_E5M2: return 1;
    default: return 0;
  }
}

kvx_status_t enqueue_write(const WritePlan &p, void *stream) {
  const int cs = dtype_size((kvx_dtype_t)p.cache_dtype);
  const int is = dtype_size((kvx_dtype_t)p.io_dtype);
  const int max_bytes = (p.conv == kConvQuant) ? 8 : 16;
  const int ge = pick_chunk(p.gk, p.gv, p.dst_k, p.dst_v, cs, p.src_k,
                            p.src_v, is, p.head_dim, max_bytes, p.block_size, p.heads);
  const int64_t row_elems = (int64_t)p.heads * p.head_dim;

  WriteArgs a;
  a.src_k = static_cast<const char *>(p.src_k);
  a.src_v = static_cast<const char *>(p.src_v);
  a.dst_k = static_cast<char *>(p.dst_k);
  a.dst_v = static_cast<char *>(p.dst_v);
  a.slots = p.slots;
  a.ksc = p.k_scale;
  a.vsc = p.v_scale;
  a.gk = to_bytes(p.gk, cs);
  a.gv = to_bytes(p.gv, cs);
  a.num_tokens = p.num_tokens;
  a.slot_is64 = p.slot_is64;
  a.block_size = p.block_size;
  a.num_blocks = p.num_blocks;
  a.head_dim = p.head_dim;
  a.nchunks = (int32_t)(row_elems / ge);
  a.chunk_elems = ge;
  a.row_bytes = (int32_t)(row_elems * is);
  a.lpt_log2 = lpt_log2_for(a.nchunks);
  const int tpw = kWave >> a.lpt_log2;
  a.num_groups = (p.num_tokens + tpw - 1) / tpw;
  const int64_t want = (a.num_groups + kWavesPerBlock - 1) / kWavesPerBlock;
  WriteLaunch wl;
  // One wave per token group up to 65536 workgroups, then a grid-stride
  // loop: on MI355X a 2048-workgroup cap made c3-sized NHD prefill writes
  // 2-4% slower (8% with blocks in ascending order).
  wl.grid = (int)(want < 65536 ? want : 65536);
  wl.tiles = plan_write_tiles(p, cs, is, &wl.wt, &wl.tile_grid, &wl.tile_lds);
  // write_flat_kernel: K and V rows hold H * D consecutive elements.  A
  // chunk count that is not a power of two (576-element MLA rows: 72) finds
  // a chunk's token by multiply-high, exact while the largest flat index
  // times nchunks stays within 2^32.
  auto row_dense = [&](const Geom &g) { return row_elems_contiguous(g, p.head_dim, p.heads); };
  a.nchunks_log2 = log2_exact(a.nchunks);
  a.nchunks_magic = a.nchunks_log2 < 0 ? magic_for(a.nchunks) : 0;
  wl.flat_grid = 0;
  const int64_t flat_total = (int64_t)p.num_tokens * a.nchunks;
  const bool flat_div_ok =
      a.nchunks_log2 >= 0 || (flat_total + kFlatThreads) * a.nchunks <= (int64_t(1) << 32);
  if (row_dense(p.gk) && row_dense(p.gv) && flat_div_ok) {
    const int64_t fg = (flat_total + kFlatThreads - 1) / kFlatThreads;
    if (grid_fits(fg, kFlatThreads)) wl.flat_grid = fg;  // else write_kernel's grid-stride loop
  }
  hipStream_t s = as_stream(stream);

  if (p.conv == kConvCopy) {
    run_write_copy(ge * cs, a, wl, s);
  } else {
    const bool e5 = p.cache_dtype == KVX_DTYPE_F8_E5M2;
    switch (p.io_dtype) {
      case KVX_DTYPE_F32:
        (e5 ? run_write_quant_e5m2_f32 : run_write_quant_e4m3_f32)(ge, a, wl, s);
        break;
      case KVX_DTYPE_F16:
        (e5 ? run_write_quant_e5m2_f16 : run_write_quant_e4m3_f16)(ge, a, wl, s);
        break;
      default:
        (e5 ? run_write_quant_e5m2_bf16 : run_write_quant_e4m3_bf16)(ge, a, wl, s);
        break;
    }
  }
  return hipGetLastError() == hipSuccess ? KVX_STATUS_OK
                                         : KVX_STATUS_INTERNAL_ERROR;
}

kvx_status_t enqueue_gather(const GatherPlan &p, void *stream) {
  const int cs = dtype_size((kvx_dtype_t)p.cache_dtype);
  const int is = dtype_size((kvx_dtype_t)p.io_dtype);
  // RAGGED gathers of caches whose block rows are contiguous take
  // gather_ragged_tile_kernel.
  const int64_t row_elems_all = (int64_t)p.heads * p.head_dim;
  auto rows_contig = [&](const Geom &g) {
    return row_elems_contiguous(g, p.head_dim, p.heads) &&
           (g.s_off == row_elems_all || p.block_size == 1);
  };
  const bool ragged_tile =
      p.format == KVX_BLOCK_TABLE_RAGGED && rows_contig(p.gk) && rows_contig(p.gv);
  const int max_bytes = p.conv != kConvDequant                               ? 16
                        : p.format == KVX_BLOCK_TABLE_RAGGED && !ragged_tile ? kRaggedDequantChunk
                                                                             : kDequantChunk;
  const void *base_k = p.src_k;
  const void *base_v = p.src_v;
  if (p.format == KVX_BLOCK_TABLE_KV_OFFSETS) {
    // Blocks start at pool + index * bytes_per_block: every such address is
    // as aligned as the OR of both pool pointers and the block pitch.
    base_k = base_v = reinterpret_cast<const void *>(
        reinterpret_cast<uintptr_t>(p.pool[0]) | reinterpret_cast<uintptr_t>(p.pool[1]) |
        (uintptr_t)p.bytes_per_block);
  }
  hipStream_t s = as_stream(stream);
  // PACKED gathers whose heads are contiguous runs of a power-of-two number
  // of whole 128-byte lines (HND, or HND beside NHD; power-of-two head
  // counts) take the flat kernel with head-run addressing instead of the LDS
  // tiles: every 16-byte load and store is then part of a whole line.
  auto head_runs = [&](const Geom &g) {
    return g.s_inner == 1 && (g.pack == p.head_dim || g.s_piece == g.pack);
  };
  const int64_t head_run_bytes = (int64_t)p.head_dim * cs;
  const bool head_run_flat =
      p.format == KVX_BLOCK_TABLE_PACKED && head_runs(p.gk) &&
      head_runs(p.gv) && !(rows_contig(p.gk) && rows_contig(p.gv)) &&
      log2_exact(p.heads) >= 0 && log2_exact(head_run_bytes) >= 0 && head_run_bytes >= 128 &&
      p.block_size >= kFlatHeadRunsMinBs;
  if (!head_run_flat) {
    // Dense blocks that are not all row-major: the transposing gather.
    TileArgs t;
    int64_t tgrid = 0;
    uint32_t tlds = 0;
    const bool dq = p.conv == kConvDequant;
    if (p.seq_count > 0 && plan_tiles(p, cs, is, dq ? kDequantChunk : 16, &t, &tgrid, &tlds)) {
      if (tgrid == 0) return KVX_STATUS_OK;
      const bool i64 = p.lens_is64 != 0;
      const bool p64 = p.indptr_is64 != 0;
      if (!dq) {
        run_tiles_copy(t, p.format, i64, p64, tgrid, tlds, s);
      } else if (p.cache_dtype == KVX_DTYPE_F8_E5M2) {
        run_tiles_dequant_e5m2(p.io_dtype, t, p.format, i64, p64, tgrid, tlds, s);
      } else {
        run_tiles_dequant_e4m3(p.io_dtype, t, p.format, i64, p64, tgrid, tlds, s);
      }
      return hipGetLastError() == hipSuccess ? KVX_STATUS_OK : KVX_STATUS_INTERNAL_ERROR;
    }
  }
  const int ge = pick_chunk(p.gk, p.gv, base_k, base_v, cs, p.dst_k,
                            p.dst_v, is, p.head_dim, max_bytes, p.block_size, p.heads);
  const int64_t row_elems = (int64_t)p.heads * p.head_dim;

  GatherArgs a;
  a.src_k = static_cast<const char *>(p.src_k);
  a.src_v = static_cast<const char *>(p.src_v);
  a.dst_k = static_cast<char *>(p.dst_k);
  a.dst_v = static_cast<char *>(p.dst_v);
  a.table = p.block_table;
  a.seq_lens = p.seq_lens;
  a.ksc = p.k_scale;
  a.vsc = p.v_scale;
  a.gk = to_bytes(p.gk, cs);
  a.gv = to_bytes(p.gv, cs);
  a.out_row_bytes = row_elems * is;
  a.index_is64 = p.index_is64;
  a.lens_is64 = p.lens_is64;
  a.indptr = p.indptr;
  a.indptr_is64 = p.indptr_is64;
  a.table_count = p.table_count;
  a.pool[0] = p.pool[0];
  a.pool[1] = p.pool[1];
  a.bytes_per_block = p.bytes_per_block;
  a.pool_blocks[0] = p.pool_blocks[0];
  a.pool_blocks[1] = p.pool_blocks[1];
  a.format = p.format;
  a.rows_per_wg = 0;
  a.ragged_tile = 0;
  a.max_blocks_per_seq = p.max_blocks_per_seq;
  const int64_t by_len =
      ((int64_t)p.max_seq_len + p.block_size - 1) / p.block_size;
  a.blocks_per_seq =
      (int32_t)(by_len < p.max_blocks_per_seq ? by_len : p.max_blocks_per_seq);
  a.max_seq_len = p.max_seq_len;
  a.block_size = p.block_size;
  a.num_blocks = p.num_blocks;
  a.head_dim = p.head_dim;
  a.nchunks = (int32_t)(row_elems / ge);
  a.chunk_elems = ge;
  a.lpt_log2 = lpt_log2_for(a.nchunks);
  // Rows of a block form one contiguous run when each row is H*D
  // consecutive elements and consecutive offsets are one row apart.
  auto rows_contiguous = [&](const Geom &g) {
    return row_elems_contiguous(g, p.head_dim, p.heads) &&
           (g.s_off == row_elems || p.block_size == 1);
  };
  a.flat = rows_contiguous(p.gk) && rows_contiguous(p.gv);
  a.cph_log2 = -1;
  if (head_run_flat) {
    a.flat = 1;
    a.cph_log2 = log2_exact(p.head_dim / ge);  // ge divides the power-of-two run
  }
  a.split_log2 = 0;
  a.fold_log2 = 0;
  a.units_per_seq = 0;
  a.nchunks_log2 = log2_exact(a.nchunks);
  a.nchunks_magic = a.nchunks_log2 < 0 ? magic_for(a.nchunks) : 0;
  a.bs_log2 = log2_exact(p.block_size);
  if (p.format != KVX_BLOCK_TABLE_PACKED) {
    // indexed formats: tiles of rows, about TILE_BYTES of each tensor's cache
    // rows.  Rows that are H*D contiguous elements (any row stride) take the
    // flat kernels, which find a chunk's row by a shift or, for chunk counts
    // that are not a power of two (DeepSeek's 576-element MLA rows: 72), by
    // a multiply-high, exact while tile chunks * nchunks <= 2^32 (so at most
    // 1024 chunks per row there); otherwise the row kernel, with at least
    // one full pass of its row groups.
    auto row_dense = [&](const Geom &g) { return row_elems_contiguous(g, p.head_dim, p.heads); };
    const bool chunks_ok = a.nchunks_log2 >= 0 || a.nchunks <= 1024;
    a.flat = row_dense(p.gk) && row_dense(p.gv) && chunks_ok;
    if (ragged_tile && chunks_ok) {
      // R rows of about kFlatTileBytes of cache per tensor: a power of
      // two <= 64 (one block id per lane) that divides block_size
      int64_t want = kFlatTileBytes / (row_elems * cs);
      int64_t r = 1;
      while (r * 2 <= want && r * 2 <= kWave && p.block_size % (r * 2) == 0) r *= 2;
      a.ragged_tile = 1;
      a.rows_per_wg = (int32_t)r;
      a.blocks_per_seq = (int32_t)(((int64_t)p.max_seq_len + r - 1) / r);
      // copies of sequences of kRaggedFoldMinUnits to kRaggedFoldMaxUnits
      // tiles: two tiles per workgroup, tile w and w + J (J workgroups per
      // sequence)
      a.units_per_seq = a.blocks_per_seq;
      if (p.conv == kConvCopy && a.blocks_per_seq >= kRaggedFoldMinUnits &&
          a.blocks_per_seq <= kRaggedFoldMaxUnits) {
        a.fold_log2 = 1;  // the kernel is built for one or two tiles
        a.blocks_per_seq = (a.blocks_per_seq + 1) >> 1;
      }
    }
    const bool ragged_copy = a.flat && p.format == KVX_BLOCK_TABLE_RAGGED && p.conv == kConvCopy;
    int64_t rows = (ragged_copy ? kRaggedCopyTileBytes : kGatherTileBytes) /
                   (row_elems * cs);
    const int64_t per_pass = a.flat ? 1 : (int64_t)kWavesPerBlock * (kWave >> a.lpt_log2);
    rows = rows < per_pass ? per_pass : rows;
    if (a.flat && p.format == KVX_BLOCK_TABLE_KV_OFFSETS) {
      // a power of two no larger than the (power-of-two) block: tiles never
      // straddle blocks
      int64_t r2 = 1;
      while (r2 * 2 <= rows && r2 * 2 <= p.block_size) r2 *= 2;
      rows = r2;
    }
    if (!a.ragged_tile) {
      a.rows_per_wg = (int32_t)rows;
      a.blocks_per_seq = (int32_t)(((int64_t)p.max_seq_len + rows - 1) / rows);
    }
  } else if (a.flat) {
    // split a block's chunks into a power-of-two number of equal ranges of
    // about kFlatTileBytes of cache per tensor, while the grid stays
    // within HIP's limits (larger ranges loop inside a workgroup)
    const int64_t chunks = (int64_t)p.block_size * a.nchunks;
    const int64_t chunk_bytes = (int64_t)ge * cs;
    const int64_t blocks = (int64_t)p.seq_count * a.blocks_per_seq;
    while ((chunks >> a.split_log2) * chunk_bytes > kFlatTileBytes &&
           ((chunks >> (a.split_log2 + 1)) << (a.split_log2 + 1)) == chunks &&
           a.split_log2 < 16 && grid_fits(blocks << (a.split_log2 + 1), kFlatThreads))
      ++a.split_log2;
    const int64_t per_seq = (int64_t)a.blocks_per_seq << a.split_log2;  // units
    if (per_seq > 0x7FFFFFFF) return KVX_STATUS_UNSUPPORTED;
    // up to 1 << fold_log2 units per workgroup, strided by the workgroups
    // per sequence (kFlatFoldLog2)
    a.units_per_seq = (int32_t)per_seq;
    if (per_seq >= kFlatFoldMinUnits && per_seq <= kFlatFoldMaxUnits) a.fold_log2 = kFlatFoldLog2;
    a.blocks_per_seq = (int32_t)((per_seq + (1 << a.fold_log2) - 1) >> a.fold_log2);
  } else if (a.bs_log2 >= 0) {
    // gather_rows_kernel: a power-of-two block's rows split into
    // 1 << split_log2 equal ranges of at least kRowsTileBytes of cache
    // rows per tensor (and one full pass of the row groups), so that big
    // blocks still give the grid enough workgroups: on MI355X (c2's lengths
    // in 256-token HND blocks, bf16) 2009 -> 1775 us per layer
    const int64_t per_pass = (int64_t)kWavesPerBlock * (kWave >> a.lpt_log2);
    int64_t want = kRowsTileBytes / (row_elems * cs);
    if (want < per_pass) want = per_pass;
    const int64_t blocks = (int64_t)p.seq_count * a.blocks_per_seq;
    while ((p.block_size >> (a.split_log2 + 1)) >= want && a.split_log2 < 16 &&
           grid_fits(blocks << (a.split_log2 + 1), kBlockThreads))
      ++a.split_log2;
    const int64_t per_seq = (int64_t)a.blocks_per_seq << a.split_log2;  // workgroups
    if (per_seq > 0x7FFFFFFF) return KVX_STATUS_UNSUPPORTED;
    a.blocks_per_seq = (int32_t)per_seq;
  }
  if (a.blocks_per_seq <= 0 || p.seq_count <= 0) return KVX_STATUS_OK;
  const int64_t grid = (int64_t)p.seq_count * a.blocks_per_seq;
  // threads per workgroup of the kernel launch_gather_typed picks
  int threads = kBlockThreads;
  if (p.format == KVX_BLOCK_TABLE_PACKED) {
    if (a.flat) threads = kFlatThreads;
  } else if (a.ragged_tile) {
    threads = kFlatThreads;
  } else if (a.flat && p.format == KVX_BLOCK_TABLE_RAGGED && p.conv == kConvCopy) {
    threads = kRaggedCopyThreads;
  }
  // one workgroup per (sequence, tile): a batch whose grid exceeds HIP's
  // limits (some 4 x 10^9 work-items) is not launched
  if (!grid_fits(grid, threads)) return KVX_STATUS_UNSUPPORTED;

  if (p.conv == kConvCopy) {
    run_gather_copy(ge * cs, a, grid, s);
  } else {
    const bool e5 = p.cache_dtype == KVX_DTYPE_F8_E5M2;
    switch (p.io_dtype) {
      case KVX_DTYPE_F32:
        (e5 ? run_gather_dequant_e5m2_f32 : run_gather_dequant_e4m3_f32)(ge, a, grid, s);
        break;
      case KVX_DTYPE_F16:
        (e5 ? run_gather_dequant_e5m2_f16 : run_gather_dequant_e4m3_f16)(ge, a, grid, s);
        break;
      default:
        (e5 ? run_gather_dequant_e5m2_bf16 : run_gather_dequant_e4m3_bf16)(ge, a, grid, s);
        break;
    }
  }
  return hipGetLastError() == hipSuccess ? KVX_STATUS_OK
                                         : KVX_STATUS_INTERNAL_ERROR;
}

}  // namespace kvx
