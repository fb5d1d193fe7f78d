// ark_ckpt.hip -- ARK checkpoint files from and to device buffers
// (include/ark_ckpt.h).
//
// The V4 format has no alignment: a 28-byte file header, then per tensor a
// 16-byte header and the raw data, so after the first tensor every data
// block starts at an arbitrary byte offset.  The kernels work in 16-byte
// chunks of the aligned side and shift the other side into place:
//
//   pack_kernel   one block per <= 4 KiB of image inside one tensor's data
//                 (the block finds its tensor in a per-tensor table);
//                 a lane owns aligned 16-byte image chunks, loads the two
//                 aligned 16-byte source blocks that cover the chunk and
//                 funnel-shifts them (v_alignbyte_b32) by the tensor's
//                 uniform misalignment.  Chunks that straddle a tensor's
//                 edge, or whose second block would pass the end of the
//                 source, go byte by byte.
//   header_kernel the file header, tensor headers and trailer, byte stores.
//   unpack_kernel one block per 2048 (fp16) or 1024 (fp32) elements of one
//                 tensor (found the same way, both file types in one
//                 launch); a lane takes
//                 16-byte units of the image (8 fp16 or 4 fp32 elements),
//                 shifts them out of two aligned loads, converts to the
//                 destination type and stores aligned.
//
// All HBM bound: 2 bytes of traffic per image byte (one read, one write).
// Files move through two pinned staging buffers, copy and file I/O
// overlapped, each chunk's file I/O split over several threads.
#include <errno.h>
#include <fcntl.h>
#include <limits.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <atomic>
#include <string>
#include <thread>
#include <vector>

#include "ark_ckpt.h"
#include "ark_common.hpp"
#include "ark_device.hpp"

namespace {

using namespace ark::dev;
using ark::fail;

constexpr uint64_t kFileHeaderV4 = 28;  // u32 magic + 3 x u64 (io.rs:453-456)
constexpr uint64_t kRecHeaderV4 = 16;   // u64 n + u64 type (io.rs:460-461, :467-468)
constexpr uint64_t kTrailerBytes = 40;  // u32 magic + u32 version + ark_opt_state
constexpr uint32_t kTrailerVersion = 1;
constexpr int kThreads = 256;  // header and check kernels
constexpr uint32_t kHintShift = 8;  // pack/unpack blocks per find_rec hint: 256
// Pack and unpack launch shapes: lanes per block, and 16-byte image chunks
// (pack) or units (unpack) per lane, kLanes * 16 bytes apart.  Measured on
// MI355X over the EKO-237M image (per call): pack is best at 256 lanes with
// one chunk per lane (0.87 ms; 64-512 lanes with one to four chunks
// 0.86-1.05 ms), unpack at 512 lanes with two units per lane (0.83 ms against
// 0.85 ms for 256 x 1 and up to 0.89 ms for the others).
constexpr int kPackLanes = 256;
constexpr int kPackChunks = 1;
constexpr uint32_t kPackSegBytes = 16u * kPackLanes * kPackChunks;  // image bytes per block
constexpr int kUnpackLanes = 512;
constexpr int kUnpackUnits = 2;
// elements per unpack block: kUnpackUnits 16-byte units of the file type per lane
constexpr uint32_t unpack_seg(uint32_t ftype) {
  return (ftype == ARK_CKPT_F16 ? 8u : 4u) * kUnpackLanes * kUnpackUnits;
}
// blocks per launch of each, so that a launch's work-items stay below 2^32
constexpr uint64_t kPackMaxBlocks = ((1ull << 32) - 1) / kPackLanes;
constexpr uint64_t kUnpackMaxBlocks = ((1ull << 32) - 1) / kUnpackLanes;

// ARK_CKPT_LAUNCH_BLOCKS=k (k >= 1) caps the blocks per pack or unpack launch
// below that (a test knob: it splits even small images over many launches,
// which must give the same bytes).
uint64_t launch_blocks(uint64_t max_blocks) {
  if (const char* env = getenv("ARK_CKPT_LAUNCH_BLOCKS")) {
    const long long v = atoll(env);
    if (v >= 1 && (uint64_t)v < max_blocks) return (uint64_t)v;
  }
  return max_blocks;
}
constexpr size_t kStageBytes = (size_t)64 << 20;      // per pinned staging buffer
static_assert(sizeof(ark_opt_state) == 32, "trailer holds a 32-byte state");

inline uint64_t esize(uint32_t t) { return t == ARK_CKPT_F16 ? 2u : 4u; }

// The bytes of a V4 image that change from one save of the same records to
// the next: the file header (global step, Adam step, record count) and the
// AMP trailer.  Passed to the header kernel by value, so a prepared table
// (ark_ckpt_plan) needs no upload per save.
constexpr uint32_t kDynBytes = (uint32_t)(kFileHeaderV4 + kTrailerBytes);
struct DynHdr {
  uint8_t bytes[kDynBytes];  // file header, then trailer
  uint32_t has_trailer;
  uint64_t trailer_off;  // image offset of the trailer
};

struct HdrPiece {  // up to 16 header bytes at an image offset
  uint64_t off;
  uint32_t len;
  uint32_t pad;
  uint8_t bytes[16];
};
static_assert(sizeof(HdrPiece) == 32, "32-byte piece");

// Per-tensor tables: block b of a launch belongs to the tensor r with
// start[r] <= b < start[r + 1] (start[] holds n_tensors + 1 prefix counts;
// a binary search over it, scalar loads that stay in the scalar cache).
struct PackRec {
  const uint8_t* src;  // the tensor's first data byte (device)
  uint64_t data_off;   // image offset of that byte
  uint64_t src_bytes;  // the tensor's data bytes
  uint32_t src_vec;    // src 16-byte aligned
  uint32_t pad;
};
static_assert(sizeof(PackRec) == 32, "32-byte descriptor");

struct UnpackRec {
  void* dst;         // the tensor's first destination element
  uint64_t src_off;  // image offset of its first element
  uint64_t n;        // elements
  uint8_t dtype;     // destination element type
  uint8_t ftype;     // file element type
  uint8_t dst_vec;   // dst 16-byte aligned
  uint8_t pad[5];
};
static_assert(sizeof(UnpackRec) == 32, "32-byte descriptor");

struct CheckDesc {  // expected tensor header at an image offset
  uint64_t hdr_off;
  uint64_t n;
  uint32_t type;
  uint32_t pad;
};

// ---- device side ------------------------------------------------------------

// Bytes [sh, sh + 16) of the 32 bytes a|b (little endian); sh in 0..15 and
// uniform across the wave, so the word selection is a scalar branch.
__device__ __forceinline__ u32x4 funnel16(const u32x4 a, const u32x4 b, uint32_t sh) {
  const uint32_t sb = sh & 3u;
  uint32_t w0, w1, w2, w3, w4;
  switch (sh >> 2) {
    case 0: w0 = a.x; w1 = a.y; w2 = a.z; w3 = a.w; w4 = b.x; break;
    case 1: w0 = a.y; w1 = a.z; w2 = a.w; w3 = b.x; w4 = b.y; break;
    case 2: w0 = a.z; w1 = a.w; w2 = b.x; w3 = b.y; w4 = b.z; break;
    default: w0 = a.w; w1 = b.x; w2 = b.y; w3 = b.z; w4 = b.w; break;
  }
  u32x4 r;
  r.x = __builtin_amdgcn_alignbyte(w1, w0, sb);
  r.y = __builtin_amdgcn_alignbyte(w2, w1, sb);
  r.z = __builtin_amdgcn_alignbyte(w3, w2, sb);
  r.w = __builtin_amdgcn_alignbyte(w4, w3, sb);
  return r;
}

__device__ __forceinline__ uint32_t ld_u8(const uint8_t* p) { return ld_g<uint8_t>(p); }
__device__ __forceinline__ void st_u8(uint8_t* p, uint32_t v) { st_g<uint8_t>(p, (uint8_t)v); }

// Threads [0, npieces) write the record headers from the uploaded pieces;
// thread npieces the file header and, when the image has one, the trailer,
// from dyn (unrolled, so every byte is read from the kernel arguments at a
// fixed offset).
__global__ __launch_bounds__(kThreads) void header_kernel(const HdrPiece* __restrict__ pieces,
                                                          uint32_t npieces, DynHdr dyn,
                                                          uint8_t* __restrict__ img) {
  const uint32_t i = blockIdx.x * kThreads + threadIdx.x;
  if (i < npieces) {
    const HdrPiece* p = pieces + i;
    const uint64_t off = p->off;
    const uint32_t len = p->len;
    for (uint32_t b = 0; b < len; ++b) st_u8(img + off + b, ld_u8(p->bytes + b));
    return;
  }
  if (i != npieces) return;
#pragma unroll
  for (uint32_t j = 0; j < kFileHeaderV4; ++j) st_u8(img + j, dyn.bytes[j]);
  if (dyn.has_trailer) {
#pragma unroll
    for (uint32_t j = 0; j < kTrailerBytes; ++j)
      st_u8(img + dyn.trailer_off + j, dyn.bytes[kFileHeaderV4 + j]);
  }
}

// The tensor that block b belongs to (see PackRec).  hint[i] is the tensor
// holding block min(i << kHintShift, blocks - 1) (make_hints), so the search
// runs between two neighbouring hints: mostly zero to two steps, where a
// search over the whole table would chain ten dependent loads per block.
__device__ __forceinline__ uint32_t find_rec(const uint32_t* __restrict__ start,
                                             const uint32_t* __restrict__ hint, uint32_t b) {
  const uint32_t i = b >> kHintShift;
  uint32_t lo = hint[i], hi = hint[i + 1] + 1;  // start[lo] <= b < start[hi]
  while (hi - lo > 1) {
    const uint32_t mid = (lo + hi) >> 1;
    if (start[mid] <= b)
      lo = mid;
    else
      hi = mid;
  }
  return lo;
}

// Block j of a tensor covers image bytes [base + j*S, base + (j+1)*S) of its
// data, base = data_off rounded down to 16, clipped to the data.
__global__ __launch_bounds__(kPackLanes) void pack_kernel(const PackRec* __restrict__ recs,
                                                          const uint32_t* __restrict__ start,
                                                          const uint32_t* __restrict__ hint,
                                                          uint8_t* __restrict__ img,
                                                          uint32_t block0) {
  const uint32_t blk = block0 + blockIdx.x;
  const uint32_t r = find_rec(start, hint, blk);
  const PackRec s = recs[r];
  const uint64_t base = s.data_off & ~15ull;
  const uint64_t end = s.data_off + s.src_bytes;
  const uint64_t c0 = base + (uint64_t)(blk - start[r]) * kPackSegBytes;
  const uint64_t seg_lo = c0 > s.data_off ? c0 : s.data_off;
  const uint64_t seg_hi = c0 + kPackSegBytes < end ? c0 + kPackSegBytes : end;
#pragma unroll
  for (int k = 0; k < kPackChunks; ++k) {
    const uint64_t c = c0 + 16ull * (uint64_t)(k * kPackLanes + threadIdx.x);
    if (c >= seg_hi) break;
    const uint64_t lo = c > seg_lo ? c : seg_lo;
    const uint64_t hi = c + 16 < seg_hi ? c + 16 : seg_hi;
    if (lo == c && hi == c + 16 && s.src_vec) {
      const uint64_t so = c - s.data_off;
      const uint64_t a0 = so & ~15ull;
      const uint32_t sh = (uint32_t)(so & 15u);
      if (sh == 0) {
        st_nt<u32x4>(img + c, ld_nt<u32x4>(s.src + a0));
        continue;
      }
      if ((sh & 3u) == 0) {  // dword aligned: one 16-byte load
        st_nt<u32x4>(img + c, (u32x4)ld_nt<u32x4_a4>(s.src + so));
        continue;
      }
      if (a0 + 32 <= s.src_bytes) {
        const u32x4 a = ld_nt<u32x4>(s.src + a0);
        const u32x4 b = ld_nt<u32x4>(s.src + a0 + 16);
        st_nt<u32x4>(img + c, funnel16(a, b, sh));
        continue;
      }
    }
    for (uint64_t b = lo; b < hi; ++b) st_u8(img + b, ld_u8(s.src + (b - s.data_off)));
  }
}

// fp16 -> fp16 through fp32 (half's to_f32, then fcvtn): every value kept,
// a signalling NaN comes back quiet.
__device__ __forceinline__ uint32_t quiet16(uint32_t h) {
  return ((h & 0x7C00u) == 0x7C00u && (h & 0x03FFu) != 0u) ? (h | 0x0200u) : h;
}
__device__ __forceinline__ uint32_t quiet16x2(uint32_t w) {
  return quiet16(w & 0xFFFFu) | (quiet16(w >> 16) << 16);
}

// One 16-byte unit of the image in file type FT, converted to dtype and
// stored at dst (aligned for the destination width).
template <uint32_t FT>
__device__ __forceinline__ void store_unit(const u32x4 v, uint32_t dtype, uint8_t* dst) {
  if constexpr (FT == ARK_CKPT_F16) {  // 8 elements
    if (dtype == ARK_CKPT_F16) {
      u32x4 r;
      r.x = quiet16x2(v.x); r.y = quiet16x2(v.y); r.z = quiet16x2(v.z); r.w = quiet16x2(v.w);
      st_nt<u32x4>(dst, r);
    } else {
      u32x4 a, b;
      a.x = f16_to_f32_bits(v.x & 0xFFFFu); a.y = f16_to_f32_bits(v.x >> 16);
      a.z = f16_to_f32_bits(v.y & 0xFFFFu); a.w = f16_to_f32_bits(v.y >> 16);
      b.x = f16_to_f32_bits(v.z & 0xFFFFu); b.y = f16_to_f32_bits(v.z >> 16);
      b.z = f16_to_f32_bits(v.w & 0xFFFFu); b.w = f16_to_f32_bits(v.w >> 16);
      st_nt<u32x4>(dst, a);
      st_nt<u32x4>(dst + 16, b);
    }
  } else {  // 4 elements
    if (dtype == ARK_CKPT_F32) {
      st_nt<u32x4>(dst, v);
    } else {
      u32x2 h;
      h.x = f32_to_f16_bits(v.x) | (f32_to_f16_bits(v.y) << 16);
      h.y = f32_to_f16_bits(v.z) | (f32_to_f16_bits(v.w) << 16);
      st_nt<u32x2>(dst, h);
    }
  }
}

template <uint32_t FT>
__device__ __forceinline__ void unpack_elem(const uint8_t* src, uint32_t dtype, uint8_t* dst) {
  if constexpr (FT == ARK_CKPT_F16) {
    const uint32_t h = ld_u8(src) | (ld_u8(src + 1) << 8);
    if (dtype == ARK_CKPT_F16)
      st_g<uint16_t>(dst, (uint16_t)quiet16(h));
    else
      st_g<uint32_t>(dst, f16_to_f32_bits(h));
  } else {
    const uint32_t x = ld_u8(src) | (ld_u8(src + 1) << 8) | (ld_u8(src + 2) << 16) |
                       (ld_u8(src + 3) << 24);
    if (dtype == ARK_CKPT_F32)
      st_g<uint32_t>(dst, x);
    else
      st_g<uint16_t>(dst, (uint16_t)f32_to_f16_bits(x));
  }
}

template <uint32_t FT>
__device__ __forceinline__ void unpack_block(const UnpackRec& s, uint64_t e_begin,
                                             const uint8_t* __restrict__ img, uint64_t img_bytes) {
  constexpr uint32_t kFs = FT == ARK_CKPT_F16 ? 2u : 4u;  // file element bytes
  constexpr uint32_t kU = 16u / kFs;                       // elements per unit
  constexpr uint32_t kSegN = unpack_seg(FT);
  constexpr int kUnits = (int)(kSegN / kU / kUnpackLanes);  // units per lane
  const uint32_t ds = s.dtype == ARK_CKPT_F16 ? 2u : 4u;
  const uint64_t src_off = s.src_off + e_begin * kFs;
  const uint32_t sh = (uint32_t)(src_off & 15u);
  const uint64_t n = s.n - e_begin < kSegN ? s.n - e_begin : kSegN;
  uint8_t* dst0 = (uint8_t*)s.dst + e_begin * ds;
#pragma unroll
  for (int k = 0; k < kUnits; ++k) {
    const uint32_t e0 = ((uint32_t)k * kUnpackLanes + threadIdx.x) * kU;
    if (e0 >= n) break;
    const uint64_t sb = src_off + (uint64_t)e0 * kFs;
    const uint64_t a0 = sb & ~15ull;
    uint8_t* dst = dst0 + (uint64_t)e0 * ds;
    if (s.dst_vec && e0 + kU <= n) {
      if (sh == 0) {
        store_unit<FT>(ld_nt<u32x4>(img + a0), s.dtype, dst);
        continue;
      }
      if ((sh & 3u) == 0) {  // dword aligned: one 16-byte load
        store_unit<FT>((u32x4)ld_nt<u32x4_a4>(img + sb), s.dtype, dst);
        continue;
      }
      if (a0 + 32 <= img_bytes) {
        const u32x4 a = ld_nt<u32x4>(img + a0);
        const u32x4 b = ld_nt<u32x4>(img + a0 + 16);
        store_unit<FT>(funnel16(a, b, sh), s.dtype, dst);
        continue;
      }
    }
    for (uint32_t j = 0; j < kU && e0 + j < n; ++j)
      unpack_elem<FT>(img + sb + (uint64_t)j * kFs, s.dtype, dst + (uint64_t)j * ds);
  }
}

// Block j of a tensor converts its elements [j*S, (j+1)*S), S = unpack_seg of
// the tensor's file type.
__global__ __launch_bounds__(kUnpackLanes) void unpack_kernel(const UnpackRec* __restrict__ recs,
                                                            const uint32_t* __restrict__ start,
                                                            const uint32_t* __restrict__ hint,
                                                            const uint8_t* __restrict__ img,
                                                            uint64_t img_bytes, uint32_t block0) {
  const uint32_t blk = block0 + blockIdx.x;
  const uint32_t r = find_rec(start, hint, blk);
  const UnpackRec s = recs[r];
  const uint64_t e_begin = (uint64_t)(blk - start[r]) * unpack_seg(s.ftype);
  if (s.ftype == ARK_CKPT_F16)
    unpack_block<ARK_CKPT_F16>(s, e_begin, img, img_bytes);
  else
    unpack_block<ARK_CKPT_F32>(s, e_begin, img, img_bytes);
}

__device__ __forceinline__ uint64_t ld_u64_bytes(const uint8_t* p) {
  uint64_t x = 0;
  for (int i = 0; i < 8; ++i) x |= (uint64_t)ld_u8(p + i) << (8 * i);
  return x;
}

// Thread i < n checks tensor header i; thread n checks the file header.  The
// smallest failing index (n for the file header) lands in *bad.
__global__ __launch_bounds__(kThreads) void check_kernel(const CheckDesc* __restrict__ d,
                                                         uint32_t n, const uint8_t* __restrict__ img,
                                                         uint32_t* __restrict__ bad) {
  const uint32_t i = blockIdx.x * kThreads + threadIdx.x;
  if (i > n) return;
  bool ok;
  if (i == n) {
    const uint32_t magic = (uint32_t)ld_u8(img) | (ld_u8(img + 1) << 8) | (ld_u8(img + 2) << 16) |
                           (ld_u8(img + 3) << 24);
    ok = magic == ARK_CKPT_MAGIC_V4 && ld_u64_bytes(img + 20) == (uint64_t)n;
  } else {
    const CheckDesc c = d[i];
    const uint64_t fn = ld_u64_bytes(img + c.hdr_off);
    const uint64_t ft = ld_u64_bytes(img + c.hdr_off + 8);
    // io.rs:534: type 0 is F16, anything else is read as F32
    ok = fn == c.n && ((ft == 0) == (c.type == ARK_CKPT_F16));
  }
  if (!ok) atomicMin(bad, i);
}

// ---- host side --------------------------------------------------------------

// The file image of a save or load (the descriptor tables take StreamBuf,
// stream-ordered allocations with no device-wide synchronisation on free).
struct DevBuf {
  void* p = nullptr;
  ~DevBuf() {
    if (p) (void)hipFree(p);
  }
};

// hint[i] = the tensor holding block min(i << kHintShift, blocks - 1), for
// i = 0 .. ceil(blocks / 2^kHintShift): the last r with start[r] <= that
// block, as find_rec defines it.  blocks >= 1.
std::vector<uint32_t> make_hints(const std::vector<uint32_t>& start, uint32_t nrec,
                                 uint64_t blocks) {
  const uint64_t nh = (blocks + (1u << kHintShift) - 1) >> kHintShift;
  std::vector<uint32_t> h((size_t)nh + 1);
  uint32_t r = 0;
  for (uint64_t i = 0; i <= nh; ++i) {
    const uint64_t b = (i << kHintShift) < blocks ? (i << kHintShift) : blocks - 1;
    while (r + 1 < nrec && start[r + 1] <= b) ++r;
    h[(size_t)i] = r;
  }
  return h;
}

using ark::StreamBuf;
struct PinBuf {
  void* p = nullptr;
  ~PinBuf() {
    if (p) (void)hipHostFree(p);
  }
};
// Waits for the stream on scope exit: declared after the buffers a queued
// copy or kernel may still use, so it runs before they are freed.
struct StreamSync {
  hipStream_t s;
  ~StreamSync() { (void)hipStreamSynchronize(s); }
};
struct FileMap {
  uint8_t* p = nullptr;
  uint64_t len = 0;
  ~FileMap() {
    if (p) (void)munmap(p, len);
  }
};
struct Fd {
  int fd = -1;
  ~Fd() {
    if (fd >= 0) ::close(fd);
  }
};

struct Layout {
  std::vector<uint64_t> hdr, data;
  uint64_t end = 0;    // first byte after the last tensor
  uint64_t total = 0;  // end + trailer
};

// Validates the record table.  One launch covers every record, so buffers a
// call writes may share no byte with each other or with what it reads:
// records_written (unpack, load) makes the records pairwise disjoint, and a
// caller's image (pack writes it, unpack reads it) must be disjoint from
// every record; records a call only reads may overlap each other.  These
// address checks come before need_device's buffer queries.
int check_records(const ark_ckpt_record* r, int32_t n, bool need_device,
                  bool records_written = false, const void* image = nullptr,
                  uint64_t image_bytes = 0) {
  if (n < 0 || (n > 0 && !r)) return fail(ARK_OPT_EINVAL, "record table is NULL or n < 0");
  std::vector<ark::Span> spans;
  for (int32_t i = 0; i < n; ++i) {
    if (r[i].dtype != ARK_CKPT_F16 && r[i].dtype != ARK_CKPT_F32)
      return fail(ARK_OPT_EINVAL, "record %d: dtype %u unknown", i, r[i].dtype);
    if (r[i].n > (1ull << 48)) return fail(ARK_OPT_EINVAL, "record %d: n too large", i);
    if (((uintptr_t)r[i].data) % esize(r[i].dtype))
      return fail(ARK_OPT_EINVAL, "record %d: data not aligned to its element", i);
    const uintptr_t lo = (uintptr_t)r[i].data;
    spans.push_back({lo, lo + r[i].n * esize(r[i].dtype), "data", i});
  }
  int rc;
  if (records_written && (rc = ark::check_disjoint(spans, {}, "record", "the call"))) return rc;
  if (image && image_bytes) {
    const uintptr_t ilo = (uintptr_t)image, ihi = ilo + image_bytes;
    for (const ark::Span& s : spans)
      if (s.lo < s.hi && s.lo < ihi && ilo < s.hi)
        return fail(ARK_OPT_EINVAL, "record %d data overlaps the image", s.idx);
  }
  if (need_device) {
    ark::BufferChecker checker;
    for (int32_t i = 0; i < n; ++i)
      if ((rc = checker.check(r[i].data, r[i].n * esize(r[i].dtype), "data", i))) return rc;
  }
  return ARK_OPT_OK;
}

Layout v4_layout(const ark_ckpt_record* r, int32_t n, const uint32_t* types, bool amp) {
  Layout L;
  L.hdr.resize((size_t)n);
  L.data.resize((size_t)n);
  uint64_t off = kFileHeaderV4;
  for (int32_t i = 0; i < n; ++i) {
    L.hdr[i] = off;
    off += kRecHeaderV4;
    L.data[i] = off;
    off += r[i].n * esize(types ? types[i] : r[i].dtype);
  }
  L.end = off;
  L.total = off + (amp ? kTrailerBytes : 0);
  return L;
}

void put_bytes(std::vector<HdrPiece>& v, uint64_t off, const uint8_t* b, uint32_t len) {
  for (uint32_t k = 0; k < len; k += 16) {
    HdrPiece p{};
    p.off = off + k;
    p.len = len - k < 16 ? len - k : 16;
    memcpy(p.bytes, b + k, p.len);
    v.push_back(p);
  }
}

template <typename T>
void le(uint8_t* dst, T v) {  // little endian, as the hosts this runs on
  memcpy(dst, &v, sizeof(T));
}

// The device tables of a V4 pack, in one host buffer laid out for one
// upload: the record-header pieces, the data descriptors, the block starts
// and the hints.  What varies per save (file header, trailer) is not here.
struct PackTables {
  std::vector<uint8_t> host;
  uint32_t npieces = 0;
  size_t recs_off = 0, start_off = 0, hint_off = 0;
  uint64_t blocks = 0;
  uint64_t trailer_off = 0;  // first byte after the last record's data
  int32_t n = 0;
};

int build_pack_tables(const ark_ckpt_record* r, int32_t n, PackTables& t) {
  const Layout L = v4_layout(r, n, nullptr, false);
  std::vector<HdrPiece> pieces;
  pieces.reserve((size_t)n);
  std::vector<PackRec> recs((size_t)n);
  std::vector<uint32_t> start((size_t)n + 1);
  uint64_t blocks = 0;
  for (int32_t i = 0; i < n; ++i) {
    uint8_t rh[kRecHeaderV4];
    le<uint64_t>(rh, r[i].n);
    le<uint64_t>(rh + 8, (uint64_t)r[i].dtype);
    put_bytes(pieces, L.hdr[i], rh, kRecHeaderV4);
    const uint64_t bytes = r[i].n * esize(r[i].dtype);
    PackRec& pr = recs[i];
    pr = PackRec{};
    pr.src = (const uint8_t*)r[i].data;
    pr.data_off = L.data[i];
    pr.src_bytes = bytes;
    pr.src_vec = ((uintptr_t)r[i].data & 15u) == 0;
    start[i] = (uint32_t)blocks;
    if (bytes) {
      const uint64_t base = L.data[i] & ~15ull;
      blocks += (L.data[i] + bytes - base + kPackSegBytes - 1) / kPackSegBytes;
    }
    if (blocks > 0x7FFFFFFFu) return fail(ARK_OPT_EINVAL, "image too large");
  }
  start[n] = (uint32_t)blocks;
  const std::vector<uint32_t> hint =
      blocks ? make_hints(start, (uint32_t)n, blocks) : std::vector<uint32_t>();
  const size_t pb = pieces.size() * sizeof(HdrPiece), rb = recs.size() * sizeof(PackRec);
  const size_t stb = start.size() * sizeof(uint32_t), hb = hint.size() * sizeof(uint32_t);
  t.host.resize(pb + rb + stb + hb);
  if (pb) memcpy(t.host.data(), pieces.data(), pb);
  if (rb) memcpy(t.host.data() + pb, recs.data(), rb);
  memcpy(t.host.data() + pb + rb, start.data(), stb);
  if (hb) memcpy(t.host.data() + pb + rb + stb, hint.data(), hb);
  t.npieces = (uint32_t)pieces.size();
  t.recs_off = pb;
  t.start_off = pb + rb;
  t.hint_off = pb + rb + stb;
  t.blocks = blocks;
  t.trailer_off = L.end;
  t.n = n;
  return ARK_OPT_OK;
}

DynHdr make_dyn(uint64_t gs, uint64_t as, int32_t n, const ark_opt_state* amp,
                uint64_t trailer_off) {
  DynHdr d{};
  le<uint32_t>(d.bytes, ARK_CKPT_MAGIC_V4);
  le<uint64_t>(d.bytes + 4, gs);
  le<uint64_t>(d.bytes + 12, as);
  le<uint64_t>(d.bytes + 20, (uint64_t)n);
  if (amp) {
    uint8_t* tr = d.bytes + kFileHeaderV4;
    le<uint32_t>(tr, ARK_CKPT_MAGIC_AMP);
    le<uint32_t>(tr + 4, kTrailerVersion);
    memcpy(tr + 8, amp, sizeof(ark_opt_state));
    d.has_trailer = 1u;
    d.trailer_off = trailer_off;
  }
  return d;
}

// Queues the header kernel and the data kernels of a pack whose tables sit
// at dtab (device, laid out as PackTables::host).
int launch_pack(const uint8_t* dtab, const PackTables& t, const DynHdr& dyn, uint8_t* img,
                hipStream_t stream) {
  const uint32_t nh = t.npieces + 1;
  hipLaunchKernelGGL(header_kernel, dim3((nh + kThreads - 1) / kThreads), dim3(kThreads), 0,
                     stream, (const HdrPiece*)dtab, t.npieces, dyn, img);
  ARK_HIP(hipGetLastError());
  // a launch's work-items stay below 2^32: images past 64 GiB take several
  const uint64_t per_launch = launch_blocks(kPackMaxBlocks);
  for (uint64_t b0 = 0; b0 < t.blocks; b0 += per_launch) {
    const uint64_t nb = t.blocks - b0 < per_launch ? t.blocks - b0 : per_launch;
    hipLaunchKernelGGL(pack_kernel, dim3((uint32_t)nb), dim3(kPackLanes), 0, stream,
                       (const PackRec*)(dtab + t.recs_off), (const uint32_t*)(dtab + t.start_off),
                       (const uint32_t*)(dtab + t.hint_off), img, (uint32_t)b0);
    ARK_HIP(hipGetLastError());
  }
  return ARK_OPT_OK;
}

// The arguments of a pack into image: the records, an image of at least the
// V4 size (with the trailer when with_amp), 16-byte aligned device memory
// that shares no byte with any record.
int check_pack(const ark_ckpt_record* records, int32_t n, bool with_amp, const void* image,
               uint64_t image_bytes) {
  // the table and the image's size and alignment first, then the device
  // queries of the records' buffers and the image
  int rc = check_records(records, n, false, false, image, image_bytes);
  if (rc) return rc;
  const Layout L = v4_layout(records, n, nullptr, with_amp);
  if (image_bytes < L.total)
    return fail(ARK_OPT_EINVAL, "image holds %llu bytes, the checkpoint needs %llu",
                (unsigned long long)image_bytes, (unsigned long long)L.total);
  if ((uintptr_t)image & 15u) return fail(ARK_OPT_EINVAL, "image not 16-byte aligned");
  if ((rc = check_records(records, n, true))) return rc;
  return ark::check_buffer(image, L.total, "image", 0);
}

// The tables of a V4 image uploaded, both kernels queued on stream and
// waited for.
int pack_image(const ark_ckpt_record* r, int32_t n, uint64_t gs, uint64_t as,
               const ark_opt_state* amp, uint8_t* img, hipStream_t stream) {
  PackTables t;
  int rc = build_pack_tables(r, n, t);
  if (rc) return rc;
  StreamBuf d;
  hipError_t e = d.alloc(t.host.size(), stream);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(ARK_OPT_ENOMEM, "hipMallocAsync(%zu) for checkpoint descriptors failed",
                t.host.size());
  }
  StreamSync sync{stream};
  ARK_HIP(hipMemcpyAsync(d.p, t.host.data(), t.host.size(), hipMemcpyHostToDevice, stream));
  if ((rc = launch_pack((const uint8_t*)d.p, t, make_dyn(gs, as, n, amp, t.trailer_off), img,
                        stream)))
    return rc;
  ARK_HIP(hipStreamSynchronize(stream));
  return ARK_OPT_OK;
}

// Unpack descriptors of every record, grouped by file type, launched and
// waited for.
int unpack_image(const uint8_t* img, uint64_t img_bytes, const ark_ckpt_record* r, int32_t n,
                 const std::vector<uint64_t>& data_off, const std::vector<uint32_t>& ftype,
                 hipStream_t stream) {
  std::vector<UnpackRec> recs((size_t)n);
  std::vector<uint32_t> start((size_t)n + 1);
  uint64_t blocks = 0;
  for (int32_t i = 0; i < n; ++i) {
    UnpackRec& u = recs[i];
    u = UnpackRec{};
    u.dst = r[i].data;
    u.src_off = data_off[i];
    u.n = r[i].n;
    u.dtype = (uint8_t)r[i].dtype;
    u.ftype = (uint8_t)ftype[i];
    u.dst_vec = ((uintptr_t)r[i].data & 15u) == 0;
    start[i] = (uint32_t)blocks;
    blocks += (r[i].n + unpack_seg(ftype[i]) - 1) / unpack_seg(ftype[i]);
    if (blocks > 0x7FFFFFFFu) return fail(ARK_OPT_EINVAL, "checkpoint too large");
  }
  start[n] = (uint32_t)blocks;
  if (blocks == 0) return ARK_OPT_OK;
  {
    // a record's buffer may be an optimizer's gradient
    std::vector<const void*> dst((size_t)n);
    std::vector<uint64_t> bytes((size_t)n);
    for (int32_t i = 0; i < n; ++i) {
      dst[i] = r[i].data;
      bytes[i] = r[i].n * (r[i].dtype == ARK_CKPT_F16 ? 2u : 4u);
    }
    ark::opt_units_invalidate(dst.data(), bytes.data(), (size_t)n);
  }
  const std::vector<uint32_t> hint = make_hints(start, (uint32_t)n, blocks);
  const size_t rb = recs.size() * sizeof(UnpackRec), stb = start.size() * sizeof(uint32_t);
  const size_t hb = hint.size() * sizeof(uint32_t);
  std::vector<uint8_t> host(rb + stb + hb);
  memcpy(host.data(), recs.data(), rb);
  memcpy(host.data() + rb, start.data(), stb);
  memcpy(host.data() + rb + stb, hint.data(), hb);
  StreamBuf d;
  hipError_t e = d.alloc(host.size(), stream);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(ARK_OPT_ENOMEM, "hipMallocAsync(%zu) for checkpoint descriptors failed",
                host.size());
  }
  StreamSync sync{stream};
  ARK_HIP(hipMemcpyAsync(d.p, host.data(), host.size(), hipMemcpyHostToDevice, stream));
  // a launch's work-items stay below 2^32: checkpoints past 128 GiB take several
  const uint64_t per_launch = launch_blocks(kUnpackMaxBlocks);
  for (uint64_t b0 = 0; b0 < blocks; b0 += per_launch) {
    const uint64_t nb = blocks - b0 < per_launch ? blocks - b0 : per_launch;
    hipLaunchKernelGGL(unpack_kernel, dim3((uint32_t)nb), dim3(kUnpackLanes), 0, stream,
                       (const UnpackRec*)d.p, (const uint32_t*)((char*)d.p + rb),
                       (const uint32_t*)((char*)d.p + rb + stb), img, img_bytes, (uint32_t)b0);
    ARK_HIP(hipGetLastError());
  }
  ARK_HIP(hipStreamSynchronize(stream));
  return ARK_OPT_OK;
}

int io_fail(const char* what, const char* path) {
  return fail(ARK_OPT_EIO, "%s %s: %s", what, path, strerror(errno));
}

// Flushes the directory holding path so a rename into it is durable.  Best
// effort: some file systems refuse fsync on a directory, and the file itself
// is complete either way.
void sync_parent_dir(const char* path) {
  std::string dir(path);
  const size_t slash = dir.find_last_of('/');
  dir = slash == std::string::npos ? std::string(".") : dir.substr(0, slash ? slash : 1);
  const int d = ::open(dir.c_str(), O_RDONLY | O_DIRECTORY | O_CLOEXEC);
  if (d < 0) return;
  (void)fsync(d);
  (void)::close(d);
}

std::atomic<uint64_t> g_tmp_counter{0};

// The file a save to path writes: path itself, or, when path is a symbolic
// link, what the chain of links names, resolved one link at a time as
// open(2) resolves it, so that a dangling link names the file to create (as
// File::create creates it, io.rs:450).  Relative link targets are taken from
// the directory of the link.  A chain of more than 40 links is left to fail
// at the open, as open(2) fails on it.
std::string save_target(const char* path) {
  std::string p(path);
  for (int hops = 0; hops < 40; ++hops) {
    struct stat st;
    if (lstat(p.c_str(), &st) != 0 || !S_ISLNK(st.st_mode)) return p;
    std::vector<char> buf((size_t)(st.st_size > 0 ? st.st_size : PATH_MAX) + 1);
    const ssize_t k = readlink(p.c_str(), buf.data(), buf.size() - 1);
    if (k < 0) return p;
    std::string link(buf.data(), (size_t)k);
    if (!link.empty() && link[0] != '/') {
      const size_t slash = p.rfind('/');
      if (slash != std::string::npos) link = p.substr(0, slash + 1) + link;
    }
    p = link;
  }
  return p;
}

int read_exact(int fd, void* buf, uint64_t len, uint64_t off, const char* path) {
  uint8_t* p = (uint8_t*)buf;
  while (len) {
    const ssize_t k = pread(fd, p, len > (1u << 30) ? (1u << 30) : len, (off_t)off);
    if (k < 0) {
      if (errno == EINTR) continue;
      return io_fail("read", path);
    }
    if (k == 0) return fail(ARK_OPT_EIO, "%s: unexpected end of file at byte %llu", path,
                            (unsigned long long)off);
    p += k;
    off += (uint64_t)k;
    len -= (uint64_t)k;
  }
  return ARK_OPT_OK;
}

// Positional write of [buf, buf + len) at file offset off, retrying short
// writes.
int pwrite_all(int fd, const void* buf, uint64_t len, uint64_t off, const char* path) {
  const uint8_t* p = (const uint8_t*)buf;
  while (len) {
    const ssize_t k = ::pwrite(fd, p, len > (1u << 30) ? (1u << 30) : len, (off_t)off);
    if (k < 0) {
      if (errno == EINTR) continue;
      return io_fail("write", path);
    }
    p += k;
    off += (uint64_t)k;
    len -= (uint64_t)k;
  }
  return ARK_OPT_OK;
}

// One staging chunk to or from the file, split over up to kIoThreads
// threads (the single-threaded copy between the page cache and a pinned
// buffer, not the GPU, bounds a checkpoint's save and load).
constexpr int kIoThreads = 16;
constexpr uint64_t kIoPiece = (uint64_t)4 << 20;  // at least 4 MiB per thread

// memcpy split over up to kIoThreads threads (into a mapped file: the page
// faults of the first touch run in parallel too).
void parallel_copy(uint8_t* dst, const void* src, uint64_t len) {
  unsigned hw = std::thread::hardware_concurrency();
  int nt = (int)((len + kIoPiece - 1) / kIoPiece);
  if (nt > kIoThreads) nt = kIoThreads;
  if (hw && nt > (int)hw) nt = (int)hw;
  if (nt <= 1) {
    memcpy(dst, src, len);
    return;
  }
  std::vector<std::thread> th;
  const uint64_t piece = (len + nt - 1) / nt;
  for (int t = 0; t < nt; ++t) {
    const uint64_t a = (uint64_t)t * piece;
    const uint64_t b = a + piece < len ? a + piece : len;
    if (a >= b) break;
    th.emplace_back([=] { memcpy(dst + a, (const uint8_t*)src + a, b - a); });
  }
  for (auto& x : th) x.join();
}

int parallel_io(bool write, int fd, void* buf, uint64_t len, uint64_t off, const char* path) {
  unsigned hw = std::thread::hardware_concurrency();
  int nt = (int)((len + kIoPiece - 1) / kIoPiece);
  if (nt > kIoThreads) nt = kIoThreads;
  if (hw && nt > (int)hw) nt = (int)hw;
  if (nt <= 1)
    return write ? pwrite_all(fd, buf, len, off, path) : read_exact(fd, buf, len, off, path);
  std::vector<int> rc((size_t)nt, ARK_OPT_OK);
  std::vector<std::string> msg((size_t)nt);
  std::vector<std::thread> th;
  const uint64_t piece = (len + nt - 1) / nt;
  for (int t = 0; t < nt; ++t) {
    const uint64_t a = (uint64_t)t * piece;
    const uint64_t b = a + piece < len ? a + piece : len;
    if (a >= b) break;
    th.emplace_back([&, t, a, b] {
      uint8_t* q = (uint8_t*)buf + a;
      rc[t] = write ? pwrite_all(fd, q, b - a, off + a, path)
                    : read_exact(fd, q, b - a, off + a, path);
      if (rc[t]) msg[t] = ark::last_error();  // the message is per thread
    });
  }
  for (auto& x : th) x.join();
  for (int t = 0; t < nt; ++t)
    if (rc[t]) return fail(rc[t], "%s", msg[t].c_str());
  return ARK_OPT_OK;
}

// Header walk of a checkpoint file (io.rs:504-671): version, steps, and per
// tensor its n, file type and data offset; checks that every tensor lies
// inside the file (the reference's read_exact fails there) and looks for the
// AMP trailer after the last one.
struct Parsed {
  ark_ckpt_info info{};
  std::vector<uint64_t> n, data;
  std::vector<uint32_t> type;
  uint64_t end = 0;
  ark_opt_state amp{};
};

int parse_file(int fd, const char* path, Parsed* P) {
  struct stat st;
  if (fstat(fd, &st) != 0) return io_fail("stat", path);
  const uint64_t size = (uint64_t)st.st_size;
  uint8_t h[28];
  int rc;
  if (size < 12) return fail(ARK_OPT_EIO, "%s: %llu bytes, too short for a checkpoint", path,
                             (unsigned long long)size);
  if ((rc = read_exact(fd, h, 12, 0, path))) return rc;
  uint32_t magic;
  memcpy(&magic, h, 4);
  ark_ckpt_info& I = P->info;
  memset(&I, 0, sizeof(I));
  I.file_bytes = size;
  uint64_t off;
  memcpy(&I.global_step, h + 4, 8);
  if (magic == ARK_CKPT_MAGIC_V4 || magic == ARK_CKPT_MAGIC_V3) {
    if ((rc = read_exact(fd, h, 16, 12, path))) return rc;
    memcpy(&I.adam_step, h, 8);
    memcpy(&I.n_tensors, h + 8, 8);
    I.version = magic == ARK_CKPT_MAGIC_V4 ? 4 : 3;
    I.has_moments = 1;
    off = 28;
  } else if (magic == ARK_CKPT_MAGIC_V2) {
    if ((rc = read_exact(fd, h, 8, 12, path))) return rc;
    memcpy(&I.n_tensors, h, 8);
    I.version = 2;
    off = 20;
  } else {
    return fail(ARK_OPT_EIO, "%s: bad magic 0x%08X (not an ARK checkpoint)", path, magic);
  }
  const uint64_t hb = I.version == 4 ? 16 : 8;
  if (I.n_tensors > (size - off) / hb)
    return fail(ARK_OPT_EIO, "%s: %llu tensors cannot fit in %llu bytes", path,
                (unsigned long long)I.n_tensors, (unsigned long long)size);
  P->n.resize(I.n_tensors);
  P->data.resize(I.n_tensors);
  P->type.resize(I.n_tensors);
  for (uint64_t i = 0; i < I.n_tensors; ++i) {
    if (off + hb > size)
      return fail(ARK_OPT_EIO, "%s: truncated at tensor %llu header", path, (unsigned long long)i);
    if ((rc = read_exact(fd, h, hb, off, path))) return rc;
    uint64_t n, t = 1;
    memcpy(&n, h, 8);
    if (hb == 16) memcpy(&t, h + 8, 8);
    const uint32_t ft = t == 0 ? ARK_CKPT_F16 : ARK_CKPT_F32;  // io.rs:534
    off += hb;
    const uint64_t bytes = n * esize(ft);
    if (n > (1ull << 48) || bytes > size - off)
      return fail(ARK_OPT_EIO, "%s: truncated in tensor %llu (n=%llu)", path,
                  (unsigned long long)i, (unsigned long long)n);
    P->n[i] = n;
    P->type[i] = ft;
    P->data[i] = off;
    off += bytes;
  }
  P->end = off;
  if (I.version == 4 && size - off >= kTrailerBytes) {
    uint8_t tr[kTrailerBytes];
    if ((rc = read_exact(fd, tr, kTrailerBytes, off, path))) return rc;
    uint32_t m, v;
    memcpy(&m, tr, 4);
    memcpy(&v, tr + 4, 4);
    if (m == ARK_CKPT_MAGIC_AMP && v == kTrailerVersion) {
      I.has_amp = 1;
      memcpy(&P->amp, tr + 8, sizeof(ark_opt_state));
    }
  }
  return ARK_OPT_OK;
}

}  // namespace

// A pack prepared once: the tables on the device, the image and stream.
struct ark_ckpt_plan {
  int device = 0;
  hipStream_t stream = nullptr;
  void* d_tables = nullptr;
  uint8_t* image = nullptr;
  bool with_amp = false;
  PackTables t;  // sizes and offsets; its host copy is dropped after the upload
};

extern "C" {

int ark_ckpt_v4_image_bytes(const ark_ckpt_record* records, int32_t n, int with_amp,
                            uint64_t* bytes) {
  if (!bytes) return fail(ARK_OPT_EINVAL, "bytes is NULL");
  int rc = check_records(records, n, false);
  if (rc) return rc;
  *bytes = v4_layout(records, n, nullptr, with_amp != 0).total;
  return ARK_OPT_OK;
}

int ark_ckpt_v4_pack(const ark_ckpt_record* records, int32_t n, uint64_t global_step,
                     uint64_t adam_step, const ark_opt_state* amp, void* image,
                     uint64_t image_bytes, void* stream) {
  const int rc = check_pack(records, n, amp != nullptr, image, image_bytes);
  if (rc) return rc;
  return pack_image(records, n, global_step, adam_step, amp, (uint8_t*)image,
                    (hipStream_t)stream);
}

int ark_ckpt_v4_pack_plan_create(const ark_ckpt_record* records, int32_t n, int with_amp,
                                 void* image, uint64_t image_bytes, void* stream,
                                 ark_ckpt_plan** out) {
  if (!out) return fail(ARK_OPT_EINVAL, "out is NULL");
  *out = nullptr;
  int rc = check_pack(records, n, with_amp != 0, image, image_bytes);
  if (rc) return rc;
  int dev = 0;
  if ((rc = ark::current_device_for(stream, &dev))) return rc;
  ark_ckpt_plan* p = new ark_ckpt_plan();
  if ((rc = build_pack_tables(records, n, p->t))) {
    delete p;
    return rc;
  }
  p->stream = (hipStream_t)stream;
  p->image = (uint8_t*)image;
  p->with_amp = with_amp != 0;
  p->device = dev;
  hipError_t e = hipMalloc(&p->d_tables, p->t.host.size());
  if (e == hipSuccess)
    e = hipMemcpy(p->d_tables, p->t.host.data(), p->t.host.size(), hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    if (p->d_tables) (void)hipFree(p->d_tables);
    delete p;
    return ark::hip_fail(e, "ark_ckpt_v4_pack_plan_create");
  }
  p->t.host.clear();
  p->t.host.shrink_to_fit();
  *out = p;
  return ARK_OPT_OK;
}

int ark_ckpt_v4_pack_plan_run(ark_ckpt_plan* p, uint64_t global_step, uint64_t adam_step,
                              const ark_opt_state* amp) {
  if (!p) return fail(ARK_OPT_EINVAL, "plan is NULL");
  if ((amp != nullptr) != p->with_amp)
    return fail(ARK_OPT_EINVAL, p->with_amp ? "the plan's image has a trailer: amp is NULL"
                                            : "the plan's image has no trailer: amp must be NULL");
  ark::DeviceGuard g(p->device);
  if (!g.ok) return fail(ARK_OPT_EHIP, "cannot select device %d", p->device);
  return launch_pack((const uint8_t*)p->d_tables, p->t,
                     make_dyn(global_step, adam_step, p->t.n, amp, p->t.trailer_off), p->image,
                     p->stream);
}

int ark_ckpt_plan_destroy(ark_ckpt_plan* p) {
  if (!p) return ARK_OPT_OK;
  int rc = ARK_OPT_OK;
  if (p->d_tables) {
    ark::DeviceGuard g(p->device);
    hipError_t e = hipFree(p->d_tables);
    if (e != hipSuccess) rc = ark::hip_fail(e, "hipFree");
  }
  delete p;
  return rc;
}

int ark_ckpt_v4_unpack(const void* image, uint64_t image_bytes, const ark_ckpt_record* records,
                       int32_t n, const uint32_t* file_types, void* stream) {
  int rc = check_records(records, n, true, true, image, image_bytes);
  if (rc) return rc;
  if (n > 0 && !file_types) return fail(ARK_OPT_EINVAL, "file_types is NULL");
  for (int32_t i = 0; i < n; ++i)
    if (file_types[i] != ARK_CKPT_F16 && file_types[i] != ARK_CKPT_F32)
      return fail(ARK_OPT_EINVAL, "file_types[%d] = %u unknown", i, file_types[i]);
  const Layout L = v4_layout(records, n, file_types, false);
  if (image_bytes < L.end)
    return fail(ARK_OPT_EINVAL, "image holds %llu bytes, the layout needs %llu",
                (unsigned long long)image_bytes, (unsigned long long)L.end);
  if ((uintptr_t)image & 15u) return fail(ARK_OPT_EINVAL, "image not 16-byte aligned");
  if ((rc = ark::check_buffer(image, image_bytes, "image", 0))) return rc;
  hipStream_t s = (hipStream_t)stream;
  // header check on the device
  std::vector<CheckDesc> cd((size_t)n);
  for (int32_t i = 0; i < n; ++i) cd[i] = CheckDesc{L.hdr[i], records[i].n, file_types[i], 0};
  // one upload: the header descriptors, then the failure index (all ones:
  // no failure)
  const size_t cb = cd.size() * sizeof(CheckDesc);
  std::vector<uint8_t> host(cb + 16, 0xFF);
  if (cb) memcpy(host.data(), cd.data(), cb);
  StreamBuf d;
  hipError_t e = d.alloc(host.size(), s);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(ARK_OPT_ENOMEM, "hipMallocAsync(%zu) for checkpoint descriptors failed",
                host.size());
  }
  StreamSync sync{s};
  uint32_t* dbad = (uint32_t*)((char*)d.p + cb);
  ARK_HIP(hipMemcpyAsync(d.p, host.data(), host.size(), hipMemcpyHostToDevice, s));
  hipLaunchKernelGGL(check_kernel, dim3((uint32_t)(n + 1 + kThreads - 1) / kThreads),
                     dim3(kThreads), 0, s, (const CheckDesc*)d.p, (uint32_t)n,
                     (const uint8_t*)image, dbad);
  ARK_HIP(hipGetLastError());
  uint32_t bad = 0;
  ARK_HIP(hipMemcpyAsync(&bad, dbad, 4, hipMemcpyDeviceToHost, s));
  ARK_HIP(hipStreamSynchronize(s));
  if (bad == (uint32_t)n)
    return fail(ARK_OPT_EIO, "image: V4 file header missing or n_tensors != %d", n);
  if (bad != 0xFFFFFFFFu)
    return fail(ARK_OPT_EIO, "image: tensor %u header does not match the record (n=%llu)", bad,
                (unsigned long long)records[bad].n);
  std::vector<uint32_t> ft(file_types, file_types + n);
  return unpack_image((const uint8_t*)image, image_bytes, records, n, L.data, ft, s);
}

int ark_ckpt_save_v4(const char* path, uint64_t global_step, uint64_t adam_step,
                     const ark_ckpt_record* records, int32_t n, const ark_opt_state* amp,
                     void* stream) {
  if (!path) return fail(ARK_OPT_EINVAL, "path is NULL");
  int rc = check_records(records, n, true);
  if (rc) return rc;
  hipStream_t s = (hipStream_t)stream;
  const Layout L = v4_layout(records, n, nullptr, amp != nullptr);
  DevBuf img;
  hipError_t e = hipMalloc(&img.p, L.total + 16);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(ARK_OPT_ENOMEM, "hipMalloc(%llu) for the checkpoint image failed",
                (unsigned long long)L.total);
  }
  if ((rc = pack_image(records, n, global_step, adam_step, amp, (uint8_t*)img.p, s))) return rc;
  const size_t stage = L.total < kStageBytes ? (size_t)L.total : kStageBytes;
  PinBuf pin[2];
  for (auto& p : pin) {
    if ((e = hipHostMalloc(&p.p, stage, hipHostMallocDefault)) != hipSuccess) {
      (void)hipGetLastError();
      return fail(ARK_OPT_ENOMEM, "hipHostMalloc(%zu) failed", stage);
    }
  }
  hipEvent_t ev[2] = {nullptr, nullptr};
  for (auto& x : ev) ARK_HIP(hipEventCreateWithFlags(&x, hipEventDisableTiming));
  struct EvGuard {
    hipEvent_t* e;
    ~EvGuard() {
      for (int i = 0; i < 2; ++i)
        if (e[i]) (void)hipEventDestroy(e[i]);
    }
  } eg{ev};
  StreamSync sync{s};
  // Written to a temporary file beside the target and renamed over it once
  // complete: a save that fails leaves no partial file (one that fallocate
  // has sized in full would pass a loader's length checks) and any earlier
  // checkpoint intact.  The temporary name is unique to this call
  // (<target>.tmp.<pid>.<n>, created with O_EXCL), so concurrent saves and a
  // user's own files never share it.  A symbolic link at path is followed, as
  // File::create follows it (io.rs:450): the link stays and the file it names
  // becomes the new file, also when the link dangles.  A new file gets mode
  // 0666 less the umask, File::create's; a file it replaces hands its mode,
  // and where permitted its owner and group, on to the new one, which
  // File::create keeps by truncating in place.  Other names (hard links) of a
  // replaced file keep the old contents: a rename cannot carry them over.
  const std::string target = save_target(path);
  std::string tmp;
  Fd f;
  for (int attempt = 0; attempt < 16 && f.fd < 0; ++attempt) {
    tmp = target + ".tmp." + std::to_string((long)getpid()) + "." +
          std::to_string(g_tmp_counter.fetch_add(1));
    f.fd = ::open(tmp.c_str(), O_RDWR | O_CREAT | O_EXCL | O_CLOEXEC, 0666);
    if (f.fd < 0 && errno != EEXIST) break;
  }
  if (f.fd < 0) return io_fail("create", tmp.c_str());
  struct TmpFile {
    const std::string& name;
    bool done = false;
    ~TmpFile() {
      if (!done) (void)::unlink(name.c_str());
    }
  } tmp_file{tmp};
  {
    struct stat old;
    if (::stat(target.c_str(), &old) == 0 && S_ISREG(old.st_mode)) {
      struct stat cur;
      if (fstat(f.fd, &cur) == 0 && (cur.st_uid != old.st_uid || cur.st_gid != old.st_gid))
        (void)fchown(f.fd, old.st_uid, old.st_gid);  // EPERM for others' files: kept ours
      if (fchmod(f.fd, old.st_mode & 07777) != 0) return io_fail("set the mode of", tmp.c_str());
    }
  }
  // Preferred: reserve the whole file, map it, and copy each chunk into the
  // mapping from several threads (writes to one file through write() are
  // serialised by the file's lock).  The reservation makes a full disk fail
  // here, with an error, instead of at a page fault.  Where reserving or
  // mapping is not supported, fall back to pwrite.
  FileMap map;
  // fallocate (not posix_fallocate, which falls back to writing zeros where
  // the file system cannot reserve): unsupported means pwrite instead.
  if (fallocate(f.fd, 0, 0, (off_t)L.total) == 0) {
    void* m = mmap(nullptr, L.total, PROT_READ | PROT_WRITE, MAP_SHARED, f.fd, 0);
    if (m != MAP_FAILED) {
      map.p = (uint8_t*)m;
      map.len = L.total;
    }
  }
  // chunk k: D2H into pin[k & 1]; while it runs, write chunk k - 1
  const uint64_t nchunks = (L.total + stage - 1) / stage;
  for (uint64_t k = 0; k <= nchunks; ++k) {
    if (k < nchunks) {
      const uint64_t off = k * stage;
      const uint64_t len = L.total - off < stage ? L.total - off : stage;
      ARK_HIP(hipMemcpyAsync(pin[k & 1].p, (char*)img.p + off, len, hipMemcpyDeviceToHost, s));
      ARK_HIP(hipEventRecord(ev[k & 1], s));
    }
    if (k > 0) {
      const uint64_t j = k - 1;
      const uint64_t off = j * stage;
      const uint64_t len = L.total - off < stage ? L.total - off : stage;
      ARK_HIP(hipEventSynchronize(ev[j & 1]));
      if (map.p)
        parallel_copy(map.p + off, pin[j & 1].p, len);
      else if ((rc = parallel_io(true, f.fd, pin[j & 1].p, len, off, tmp.c_str())))
        return rc;
    }
  }
  if (map.p && munmap(map.p, map.len) != 0) return io_fail("unmap", tmp.c_str());
  map.p = nullptr;
  // The data reaches the disk before the rename does, so a crash of the
  // machine cannot leave path naming a file whose pages were never written.
  if (fdatasync(f.fd) != 0) return io_fail("flush", tmp.c_str());
  const int fd = f.fd;
  f.fd = -1;
  if (::close(fd) != 0) return io_fail("close", tmp.c_str());
  if (::rename(tmp.c_str(), target.c_str()) != 0) return io_fail("rename to", target.c_str());
  tmp_file.done = true;
  sync_parent_dir(target.c_str());
  return ARK_OPT_OK;
}

int ark_ckpt_probe(const char* path, ark_ckpt_info* info, uint64_t* n_out, uint32_t* type_out,
                   int32_t max) {
  if (!path) return fail(ARK_OPT_EINVAL, "path is NULL");
  Fd f;
  f.fd = ::open(path, O_RDONLY | O_CLOEXEC);
  if (f.fd < 0) return io_fail("open", path);
  Parsed P;
  int rc = parse_file(f.fd, path, &P);
  if (rc) return rc;
  if (info) *info = P.info;
  for (int32_t i = 0; i < max && (uint64_t)i < P.info.n_tensors; ++i) {
    if (n_out) n_out[i] = P.n[i];
    if (type_out) type_out[i] = P.type[i];
  }
  return ARK_OPT_OK;
}

int ark_ckpt_load(const char* path, const ark_ckpt_record* records, int32_t n,
                  ark_ckpt_info* info, ark_opt_state* amp, void* stream) {
  if (!path) return fail(ARK_OPT_EINVAL, "path is NULL");
  int rc = check_records(records, n, true, true);
  if (rc) return rc;
  Fd f;
  f.fd = ::open(path, O_RDONLY | O_CLOEXEC);
  if (f.fd < 0) return io_fail("open", path);
  Parsed P;
  if ((rc = parse_file(f.fd, path, &P))) return rc;
  if (P.info.n_tensors != (uint64_t)n)
    return fail(ARK_OPT_EINVAL, "%s holds %llu tensors, %d records given", path,
                (unsigned long long)P.info.n_tensors, n);
  for (int32_t i = 0; i < n; ++i)
    if (P.n[i] != records[i].n)
      return fail(ARK_OPT_EINVAL, "%s: tensor %d has n=%llu, record %d has n=%llu", path, i,
                  (unsigned long long)P.n[i], i, (unsigned long long)records[i].n);
  hipStream_t s = (hipStream_t)stream;
  const uint64_t total = P.end;
  DevBuf img;
  hipError_t e = hipMalloc(&img.p, total + 16);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(ARK_OPT_ENOMEM, "hipMalloc(%llu) for the checkpoint image failed",
                (unsigned long long)total);
  }
  const size_t stage = total < kStageBytes ? (size_t)total : kStageBytes;
  PinBuf pin[2];
  for (auto& p : pin) {
    if ((e = hipHostMalloc(&p.p, stage ? stage : 16, hipHostMallocDefault)) != hipSuccess) {
      (void)hipGetLastError();
      return fail(ARK_OPT_ENOMEM, "hipHostMalloc(%zu) failed", stage);
    }
  }
  hipEvent_t ev[2] = {nullptr, nullptr};
  for (auto& x : ev) ARK_HIP(hipEventCreateWithFlags(&x, hipEventDisableTiming));
  struct EvGuard {
    hipEvent_t* e;
    ~EvGuard() {
      for (int i = 0; i < 2; ++i)
        if (e[i]) (void)hipEventDestroy(e[i]);
    }
  } eg{ev};
  StreamSync sync{s};
  // chunk k: read into pin[k & 1] once its previous copy (chunk k - 2) is
  // done, then H2D on the stream
  const uint64_t nchunks = stage ? (total + stage - 1) / stage : 0;
  for (uint64_t k = 0; k < nchunks; ++k) {
    const uint64_t off = k * stage;
    const uint64_t len = total - off < stage ? total - off : stage;
    if (k >= 2) ARK_HIP(hipEventSynchronize(ev[k & 1]));
    if ((rc = parallel_io(false, f.fd, pin[k & 1].p, len, off, path))) return rc;
    ARK_HIP(hipMemcpyAsync((char*)img.p + off, pin[k & 1].p, len, hipMemcpyHostToDevice, s));
    ARK_HIP(hipEventRecord(ev[k & 1], s));
  }
  if ((rc = unpack_image((const uint8_t*)img.p, total, records, n, P.data, P.type, s)))
    return rc;
  if (info) *info = P.info;
  if (amp && P.info.has_amp) *amp = P.amp;
  return ARK_OPT_OK;
}

}  // extern "C"
