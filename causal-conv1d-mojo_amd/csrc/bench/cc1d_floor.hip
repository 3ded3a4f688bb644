// cc1d_floor.hip -- bandwidth floors for bench.py (measurement only; the
// product library does not contain or call these kernels).
//
// Each kernel moves the bytes of one configuration with no arithmetic, so
// its time is what HBM and the launch cost for that access pattern on this
// GPU. Every store writes a value that differs from what was loaded (bits
// flipped), so no store can be dropped as a no-op. Every access that is not a
// partial-line read-modify-write is non-temporal: on this GPU that is the
// faster form for data touched once (the C2 one-row-per-wavefront streams
// 40.2 against 43.4 us with cached loads, the C4a scattered rows 5.2 against
// 6.5 us); the circular decode's state chunks stay cached, as in the kernel.
//
//   cc1d_floor_copy   -- a plain streaming copy of n 16-byte vectors: one
//                        vector per lane, 64-thread blocks (the fastest shape
//                        measured for ~10 MB copies).
//   cc1d_floor_rows   -- the scattered-row pattern of the linear decode
//                        update: for each batch entry b, read x row b and
//                        pool row idx[b], write out row b and pool row idx[b]
//                        back in place; one wavefront per 64 x vectors and
//                        the 64 * R state vectors of the same channels, all
//                        accesses coalesced.
//   cc1d_floor_tiles  -- the channel-last backward's pattern: two tensors of
//                        rows (time steps) of row_bytes are read and a third
//                        written (out = x ^ g ^ 1), a wavefront taking
//                        `rows` consecutive rows of a seg-byte column slice
//                        (seg 256: a dword per lane, 16 rows, the channel-
//                        last kernel's shape; seg 1024: 16 bytes per lane, 4
//                        rows; seg 4096: 4 x 16 bytes per lane, one row, the
//                        channel-first kernel's shape).
//   cc1d_floor_walk   -- the channel-last backward's walk: x and g read, out
//                        = x ^ g ^ 1 written, a wavefront walking 128 rows of
//                        a 256-byte column slice in 4-row chunks with the
//                        next chunk's loads in flight (bwd_clw's loop, its
//                        grid and block shape, no arithmetic).
//   cc1d_floor_chunks -- the circular decode update's pattern: per (b, c),
//                        read and write back `chunks` consecutive 16-byte
//                        chunks of state line (idx[b], c) starting at chunk
//                        cs[b] mod line_chunks (wrapping), and read x / write
//                        out `xwords` dwords. With gran > 1 the whole aligned
//                        granules of gran chunks (4: the 64-byte sectors, 8:
//                        the 128-byte line) that hold those chunks are read
//                        and written back instead, so no partial granule is
//                        written.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

namespace {

__device__ __forceinline__ u32x4 flip(u32x4 v) {
    const u32x4 one = {1u, 1u, 1u, 1u};
    return v ^ one;
}

__global__ void __launch_bounds__(64) floor_copy(const u32x4* __restrict__ src, u32x4* __restrict__ dst, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 64 + threadIdx.x;
    if (i < n) __builtin_nontemporal_store(flip(__builtin_nontemporal_load(&src[i])), &dst[i]);
}

// one wavefront per (entry, group of 64 x vectors): lane l moves x vector l
// and state vectors l, l+64, ..., l+64(R-1) of the group's state span
// (grid: groups x batch entries, so no division). Every access is
// unconditional, at a clamped in-bounds address (a lane past the end reads
// and writes the last vector again, with the same value as its owner), so the
// compiler can neither sink a load into a branch nor serialise the loads:
// x first, then the index as a scalar load behind a scheduling fence, then
// the state loads, and the stores behind a second fence. An index outside
// [0, pool_rows) is clamped to row 0 (bench.py passes permutations only).
template <int R>
__global__ void __launch_bounds__(64) floor_rows(const u32x4* __restrict__ x, u32x4* __restrict__ out,
                                                 u32x4* __restrict__ pool, const int32_t* __restrict__ idx,
                                                 uint32_t xvec, uint32_t pool_row_vec, int32_t pool_rows) {
    const int lane = threadIdx.x;
    const uint32_t b = blockIdx.y;
    const uint32_t g = blockIdx.x;
    const uint32_t xi = min(g * 64 + lane, xvec - 1);
    const u32x4 xv = __builtin_nontemporal_load(&x[(size_t)b * xvec + xi]);
    __builtin_amdgcn_sched_barrier(0);
    const int32_t r = *(const __attribute__((address_space(4))) int32_t*)(idx + b);
    u32x4* sr = pool + (size_t)(r >= 0 && r < pool_rows ? r : 0) * pool_row_vec + g * 64 * R;
    const uint32_t nsv = (xvec - g * 64) * R;  // state vectors left in this row from the group's start
    u32x4 sv[R];
#pragma unroll
    for (int j = 0; j < R; ++j) sv[j] = __builtin_nontemporal_load(&sr[min((uint32_t)(j * 64 + lane), nsv - 1)]);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_nontemporal_store(flip(xv), &out[(size_t)b * xvec + xi]);
#pragma unroll
    for (int j = 0; j < R; ++j) __builtin_nontemporal_store(flip(sv[j]), &sr[min((uint32_t)(j * 64 + lane), nsv - 1)]);
}

__global__ void __launch_bounds__(256) floor_chunks(const uint32_t* __restrict__ x, uint32_t* __restrict__ out,
                                                    u32x4* __restrict__ pool, const int32_t* __restrict__ idx,
                                                    const int32_t* __restrict__ cs, int64_t batch, int64_t dim,
                                                    int64_t line_chunks, int64_t pool_row_chunks, int64_t pool_rows,
                                                    int chunks, int xwords, int gran) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= batch * dim) return;
    const int64_t b = t / dim;
    const int64_t c = t - b * dim;
    uint32_t xv[4];
    for (int i = 0; i < xwords; ++i) xv[i] = __builtin_nontemporal_load(&x[t * xwords + i]);
    const int32_t row = idx[b];
    if (row < 0 || row >= pool_rows) return;
    int64_t k = cs[b] % line_chunks;
    if (k < 0) k += line_chunks;
    u32x4* line = pool + (int64_t)row * pool_row_chunks + c * line_chunks;
    // the chunks moved: [k, k + chunks), or the granules of gran chunks holding them
    int n = chunks;
    if (gran > 1) {
        const bool two = gran < line_chunks && (k % gran) + chunks > gran;
        k -= k % gran;
        n = two ? 2 * gran : gran;
    }
    u32x4 v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j)
        if (j < n) v[j] = line[(k + j) % line_chunks];
    for (int i = 0; i < xwords; ++i) __builtin_nontemporal_store(xv[i] ^ 1u, &out[t * xwords + i]);
#pragma unroll
    for (int j = 0; j < 16; ++j)
        if (j < n) line[(k + j) % line_chunks] = flip(v[j]);
}

// grid: (slices per row) x (row tiles / 4), 4 wavefronts per block on
// consecutive row tiles of one slice; a lane moves VPL vectors of NB bytes
// per row (vector v at byte (v * 64 + lane) * NB of the slice); all loads
// first, then all stores
template <int NB, int VPL, int ROWS>
__global__ void __launch_bounds__(256) floor_tiles(const char* __restrict__ x, const char* __restrict__ g,
                                                   char* __restrict__ out, int64_t row_bytes, int nslice) {
    typedef typename std::conditional<NB == 16, u32x4, uint32_t>::type V;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int slice = blockIdx.x % nslice;
    const int64_t tile = (int64_t)(blockIdx.x / nslice) * 4 + wave;
    const int64_t base = tile * ROWS * row_bytes + (int64_t)slice * 64 * NB * VPL + lane * NB;
    V xv[ROWS][VPL], gv[ROWS][VPL];
#pragma unroll
    for (int r = 0; r < ROWS; ++r)
#pragma unroll
        for (int v = 0; v < VPL; ++v) {
            xv[r][v] = __builtin_nontemporal_load(reinterpret_cast<const V*>(x + base + r * row_bytes + v * 64 * NB));
            gv[r][v] = __builtin_nontemporal_load(reinterpret_cast<const V*>(g + base + r * row_bytes + v * 64 * NB));
        }
#pragma unroll
    for (int r = 0; r < ROWS; ++r)
#pragma unroll
        for (int v = 0; v < VPL; ++v)
            __builtin_nontemporal_store(xv[r][v] ^ gv[r][v] ^ (V)1u,
                                        reinterpret_cast<V*>(out + base + r * row_bytes + v * 64 * NB));
}

// The channel-last backward's walk without its arithmetic: a wavefront walks
// R consecutive rows of a 256-byte column slice (a dword per lane) in G-row
// chunks, the next chunk's loads issued before the current one's stores
// (two chunk buffers), a scheduling fence after each row; WPB wavefronts per
// block take consecutive runs of one slice (grid: slices fastest, then run
// groups), as bwd_clw's blocks do.
template <int G, int R, int WPB>
__global__ void __launch_bounds__(64 * WPB) floor_walk(const char* __restrict__ x, const char* __restrict__ g,
                                                       char* __restrict__ out, uint32_t row_bytes, uint32_t nslice) {
    constexpr int NCH = R / G;
    static_assert(R % (2 * G) == 0, "chunks in pairs");
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t slice = __builtin_amdgcn_readfirstlane(blockIdx.x % nslice);
    const uint32_t run = __builtin_amdgcn_readfirstlane(blockIdx.x / nslice) * WPB + wave;
    const size_t base = (size_t)run * R * row_bytes + slice * 256;
    const char* xb = x + base;
    const char* gb = g + base;
    char* ob = out + base;
    const uint32_t lo = lane * 4;
    uint32_t cx[2][G], cg[2][G];
    auto load = [&](int c, int buf) {
#pragma unroll
        for (int j = 0; j < G; ++j) {
            const uint32_t off = (uint32_t)(c * G + j) * row_bytes + lo;
            cx[buf][j] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(xb + off));
            cg[buf][j] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(gb + off));
        }
    };
    auto rows = [&](int c, int buf) {
#pragma unroll
        for (int j = 0; j < G; ++j) {
            const uint32_t off = (uint32_t)(c * G + j) * row_bytes + lo;
            __builtin_nontemporal_store(cx[buf][j] ^ cg[buf][j] ^ 1u, reinterpret_cast<uint32_t*>(ob + off));
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    load(0, 0);
#pragma unroll 1
    for (int c = 0; c < NCH; c += 2) {
        load(c + 1, 1);
        rows(c, 0);
        if (c + 2 < NCH) load(c + 2, 0);
        rows(c + 1, 1);
    }
}

bool launched() { return hipGetLastError() == hipSuccess; }

}  // namespace

extern "C" {

// 0 on success, -1 on a bad argument, -2 if the launch failed
int cc1d_floor_copy(const void* src, void* dst, int64_t n16, void* stream) {
    if (n16 < 0 || (n16 > 0 && (src == nullptr || dst == nullptr))) return -1;
    if (n16 == 0) return 0;
    floor_copy<<<dim3((unsigned)((n16 + 63) / 64)), 64, 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<const u32x4*>(src), static_cast<u32x4*>(dst), n16);
    return launched() ? 0 : -2;
}

// x, out: (batch, xvec) 16-byte vectors; pool: pool_rows rows of pool_row_vec
// vectors, of which the first xvec * ratio are the state span; idx: (batch,)
// rows in [0, pool_rows) (others are clamped to row 0)
int cc1d_floor_rows(const void* x, void* out, void* pool, const int32_t* idx, int64_t batch, int64_t xvec,
                    int64_t pool_row_vec, int64_t pool_rows, int ratio, void* stream) {
    if (batch < 0 || batch > 65535 || xvec < 0 || ratio < 1 || ratio > 4 || pool_row_vec < xvec * ratio ||
        pool_row_vec >= ((int64_t)1 << 32) || pool_rows >= ((int64_t)1 << 31))
        return -1;
    if (batch == 0 || xvec == 0) return 0;
    if (x == nullptr || out == nullptr || pool == nullptr || idx == nullptr) return -1;
    const dim3 grid((unsigned)((xvec + 63) / 64), (unsigned)batch);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const u32x4* xv = static_cast<const u32x4*>(x);
    u32x4* ov = static_cast<u32x4*>(out);
    u32x4* pv = static_cast<u32x4*>(pool);
    switch (ratio) {
    case 1: floor_rows<1><<<grid, 64, 0, s>>>(xv, ov, pv, idx, (uint32_t)xvec, (uint32_t)pool_row_vec, (int32_t)pool_rows); break;
    case 2: floor_rows<2><<<grid, 64, 0, s>>>(xv, ov, pv, idx, (uint32_t)xvec, (uint32_t)pool_row_vec, (int32_t)pool_rows); break;
    case 3: floor_rows<3><<<grid, 64, 0, s>>>(xv, ov, pv, idx, (uint32_t)xvec, (uint32_t)pool_row_vec, (int32_t)pool_rows); break;
    default: floor_rows<4><<<grid, 64, 0, s>>>(xv, ov, pv, idx, (uint32_t)xvec, (uint32_t)pool_row_vec, (int32_t)pool_rows); break;
    }
    return launched() ? 0 : -2;
}

// x, g, out: `rows` rows of row_bytes each (16-byte aligned); seg 256
// (16 rows per wavefront), 1024 (4 rows) or 4096 (1 row); row_bytes a
// multiple of seg and rows a multiple of 4 * rows per wavefront
int cc1d_floor_tiles(const void* x, const void* g, void* out, int64_t rows, int64_t row_bytes, int seg,
                     void* stream) {
    const int per = seg == 256 ? 16 : (seg == 1024 ? 4 : 1);
    if ((seg != 256 && seg != 1024 && seg != 4096) || rows < 0 || row_bytes <= 0 || row_bytes % seg ||
        rows % (4 * per))
        return -1;
    if (rows == 0) return 0;
    if (x == nullptr || g == nullptr || out == nullptr) return -1;
    const int nslice = (int)(row_bytes / seg);
    const int64_t blocks = nslice * (rows / (4 * per));
    if (blocks >= ((int64_t)1 << 31)) return -1;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const char* xc = static_cast<const char*>(x);
    const char* gc = static_cast<const char*>(g);
    char* oc = static_cast<char*>(out);
    if (seg == 256) floor_tiles<4, 1, 16><<<dim3((unsigned)blocks), 256, 0, s>>>(xc, gc, oc, row_bytes, nslice);
    else if (seg == 1024) floor_tiles<16, 1, 4><<<dim3((unsigned)blocks), 256, 0, s>>>(xc, gc, oc, row_bytes, nslice);
    else floor_tiles<16, 4, 1><<<dim3((unsigned)blocks), 256, 0, s>>>(xc, gc, oc, row_bytes, nslice);
    return launched() ? 0 : -2;
}

// x, g, out: `rows` rows of row_bytes each (4-byte aligned); row_bytes a
// multiple of 256 below 2^32 / 128, rows a multiple of 1024 (8 runs of 128)
int cc1d_floor_walk(const void* x, const void* g, void* out, int64_t rows, int64_t row_bytes, void* stream) {
    constexpr int G = 4, R = 128, WPB = 8;
    if (rows < 0 || row_bytes <= 0 || row_bytes % 256 || row_bytes * R >= ((int64_t)1 << 32) || rows % (R * WPB))
        return -1;
    if (rows == 0) return 0;
    if (x == nullptr || g == nullptr || out == nullptr) return -1;
    const int64_t nslice = row_bytes / 256;
    const int64_t blocks = nslice * (rows / (R * WPB));
    if (blocks >= ((int64_t)1 << 31)) return -1;
    floor_walk<G, R, WPB><<<dim3((unsigned)blocks), 64 * WPB, 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<const char*>(x), static_cast<const char*>(g), static_cast<char*>(out), (uint32_t)row_bytes,
        (uint32_t)nslice);
    return launched() ? 0 : -2;
}

// pool: pool_rows rows of pool_row_chunks 16-byte chunks, dim lines of
// line_chunks chunks each; x, out: (batch, dim) items of xwords dwords; chunks
// in {1, 2}; xwords in 1..4; gran 1 (the chunks themselves) or 4 / 8 (whole
// granules, dividing line_chunks, at most 8); idx entries outside
// [0, pool_rows) are skipped
int cc1d_floor_chunks(const void* x, void* out, void* pool, const int32_t* idx, const int32_t* cs, int64_t batch,
                      int64_t dim, int64_t line_chunks, int64_t pool_row_chunks, int64_t pool_rows, int chunks,
                      int xwords, int gran, void* stream) {
    if (batch < 0 || dim < 0 || line_chunks < 2 || chunks < 1 || chunks > 2 || xwords < 1 || xwords > 4 ||
        pool_row_chunks < dim * line_chunks || (gran != 1 && gran != 4 && gran != 8) || line_chunks % gran)
        return -1;
    if (batch == 0 || dim == 0) return 0;
    if (x == nullptr || out == nullptr || pool == nullptr || idx == nullptr || cs == nullptr) return -1;
    floor_chunks<<<dim3((unsigned)((batch * dim + 255) / 256)), 256, 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<const uint32_t*>(x), static_cast<uint32_t*>(out), static_cast<u32x4*>(pool), idx, cs, batch, dim,
        line_chunks, pool_row_chunks, pool_rows, chunks, xwords, gran);
    return launched() ? 0 : -2;
}

}  // extern "C"
