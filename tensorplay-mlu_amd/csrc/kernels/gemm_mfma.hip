// Matrix-core GEMM for gfx950 (CDNA4), and the dispatch between it and the
// general kernel (gemm.hip).
//
// C[b] = alpha * op(A[b]) op(B[b]) + beta * Cin[b] with float32
// accumulation on MFMA:
//   * bfloat16 / float16: v_mfma_f32_32x32x16_{bf16,f16} -- each lane feeds
//     8 consecutive k of one row of A and of one column of B;
//   * float32: v_mfma_f32_32x32x2_f32 -- each lane feeds one k; a 16-byte
//     LDS read gives a lane 4 consecutive k that feed 4 back-to-back MFMAs
//     (lane half h supplies k = 4h + j to MFMA j, for A and B alike, so the
//     pairing of A and B elements is exact whatever order the sum takes).
// Kernels, tried in this order:
//   * 16-bit operands, K of 64 or 128, M and N multiples of 256, at least
//     one 256 x 256 tile per CU: `smallk` below -- all of K loaded at once,
//     one barrier, the stores of one 32 x 32 tile overlapping the MFMAs of
//     the next (attention-sized bmm).
//   * 16-bit operands, M and N multiples of 256, K of 128, at least one
//     256 x 256 tile per CU: `big` below -- four waves of 128 x 128 (eight
//     of 128 x 64 when K <= 256), operand
//     tiles loaded straight into LDS by buffer loads and read back with
//     ds_read_b128 (K-major operands) or ds_read_b64_tr_b16 (transposed
//     views, read in place); no bounds checks anywhere in the K loop.
//   * other 16-bit products with a 256 x 256 tile per CU: 256 x 256 with
//     8 waves (2 x 4, each wave a 128 x 64 patch of 4 x 2 MFMA tiles of
//     32 x 32).
//   * everything else: 128 x 128 with 4 waves (2 x 2, each 64 x 64); a
//     product too small for those tiles to reach a quarter of the CUs
//     (float32: even split over K) takes 64 x 64 with 2 waves (each
//     32 x 64).
// The last two advance K BK at a time through two LDS stages: while the
// waves multiply out of one stage, the next K tile is written into the
// other and the one after is already in flight from global memory, so each
// K step needs a single barrier.  Operands sit in LDS K-major ([row][k],
// rows padded by 16 bytes so the 16-byte fragment reads of 16 consecutive
// rows hit distinct banks).  An operand stored K-major in memory is copied
// with 16-byte loads; a 16-bit one stored with its M (or N) axis contiguous
// is loaded as V x 4 blocks (V along M/N, 4 along K) and transposed in
// registers before its LDS store, a float32 one is kept as it lies
// ([k][row] tiles, read back one float at a time).  All kernels number their
// tiles so each of the 8 XCDs walks a contiguous range in groups of 8 tile
// rows, keeping an XCD's A and B panels hot in its own L2.  A float32
// product of one matrix with too few tiles to fill the CUs is split over K
// (launch_splitk).

#include <type_traits>
#include <utility>

#include "device_common.h"
#include "gemm.h"
#include "../allocator.h"
#include "../common.h"
#include "../runtime.h"
#include "tp_amd_kernels.h"

namespace tp_amd {

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

template <typename T>
struct Mfma;

template <>
struct Mfma<bf16_t> {
    static constexpr int V = 8;     // elements per 16-byte vector
    static constexpr int BK = 64;   // K per LDS tile
    static constexpr int KSUB = 16; // K per fragment read
    __device__ __forceinline__ static f32x16 mma(const uint4& a, const uint4& b, f32x16 c) {
        bf16x8 av, bv;
        __builtin_memcpy(&av, &a, 16);
        __builtin_memcpy(&bv, &b, 16);
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, c, 0, 0, 0);
    }
};

template <>
struct Mfma<f16_t> {
    static constexpr int V = 8;
    static constexpr int BK = 64;
    static constexpr int KSUB = 16;
    __device__ __forceinline__ static f32x16 mma(const uint4& a, const uint4& b, f32x16 c) {
        f16x8 av, bv;
        __builtin_memcpy(&av, &a, 16);
        __builtin_memcpy(&bv, &b, 16);
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bv, c, 0, 0, 0);
    }
};

template <>
struct Mfma<float> {
    static constexpr int V = 4;
    static constexpr int BK = 32;
    static constexpr int KSUB = 8;
    __device__ __forceinline__ static f32x16 mma(const uint4& a, const uint4& b, f32x16 c) {
        c = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.x), __uint_as_float(b.x), c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.y), __uint_as_float(b.y), c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.z), __uint_as_float(b.z), c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.w), __uint_as_float(b.w), c, 0, 0, 0);
        return c;
    }
};

constexpr int kGroupM = 8;

// Stores of C bypass the caches' normal retention (non-temporal): a large
// product's output then does not evict the A and B panels later tiles read
// (bf16 linear 8192 x 4096 x 11008: 704-713 -> 656-670 us).
template <typename S>
__device__ __forceinline__ void put_c(S* dst, S v) {
    __builtin_nontemporal_store(v, dst);
}

__device__ __forceinline__ uint32_t component(const uint4& v, int i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// One operand's tile loader: R rows (M or N) x BK, into LDS [R][BK + pad].
// KMAJOR: element (r, k) at X[r * ld + k]; otherwise at X[k * ld + r].
// A float32 operand with its M (or N) axis contiguous (KROWS) is copied as it
// lies instead, [BK][R + 8]: 16-byte loads along the row, 32 lanes a row, and
// 16-byte LDS stores; the fragment reads then take a lane's 4 consecutive k
// as 4 single-float reads, the two lane halves 4 rows apart, which the pad of
// 8 floats puts on the other half of the 64 banks.  (Transposing 4 x 4
// blocks in registers before a K-major store, as the 16-bit types do, left
// the float32 NN and TN products waiting 7-10x longer than NT: 4096^3 NN
// 1469 us, TN 1606 us, NT 1261 us.)
template <typename T, int R, bool KMAJOR, int THREADS>
struct TileLoader {
    using S = typename Elem<T>::storage;
    static constexpr int V = Mfma<T>::V;
    static constexpr int BK = Mfma<T>::BK;
    static constexpr int LDS_STRIDE = BK + 16 / sizeof(S);  // elements per LDS row
    static constexpr bool KROWS = !KMAJOR && sizeof(S) == 4;
    static constexpr int KR_STRIDE = R + 8;                  // KROWS: elements per LDS row (one k)
    static_assert(!KROWS || BK * KR_STRIDE <= R * LDS_STRIDE, "KROWS tile fits the K-major space");
    // K-major: R * BK / V vectors; MN-major: (R / V) * (BK / 4) units of 4
    // vectors (V along M/N by 4 along K).
    static constexpr int kLoads = (KMAJOR ? R * BK / V : (R / V) * (BK / 4) * 4) / THREADS;
    static constexpr int kUnits = kLoads / 4;  // MN-major units per thread
    static_assert(kLoads * THREADS == (KMAJOR ? R * BK / V : (R / V) * (BK / 4) * 4) &&
                      (KMAJOR || kUnits * 4 == kLoads),
                  "tile shape and thread count disagree");
    uint4 reg[kLoads];

    __device__ __forceinline__ void load(const S* X, int64_t ld, int64_t r0, int64_t rows,
                                         int64_t k0, int64_t K) {
        const int tid = threadIdx.x;
        if constexpr (KROWS) {
#pragma unroll
            for (int i = 0; i < kLoads; ++i) {
                const int v = tid + i * THREADS;
                const int k = v / (R / V), c = v % (R / V);
                const int64_t gr = r0 + c * V, gk = k0 + k;
                if (gr < rows && gk < K) {
                    reg[i] = *reinterpret_cast<const uint4*>(X + gk * ld + gr);
                } else {
                    reg[i] = make_uint4(0, 0, 0, 0);
                }
            }
        } else if constexpr (KMAJOR) {
#pragma unroll
            for (int i = 0; i < kLoads; ++i) {
                const int v = tid + i * THREADS;
                const int r = v / (BK / V), kc = v % (BK / V);
                const int64_t gr = r0 + r, gk = k0 + kc * V;
                if (gr < rows && gk < K) {
                    reg[i] = *reinterpret_cast<const uint4*>(X + gr * ld + gk);
                } else {
                    reg[i] = make_uint4(0, 0, 0, 0);
                }
            }
        } else {
#pragma unroll
            for (int u = 0; u < kUnits; ++u) {
                const int unit = tid + u * THREADS;
                const int kb = unit % (BK / 4), rb = unit / (BK / 4);
                const int64_t gr = r0 + rb * V;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int64_t gk = k0 + kb * 4 + i;
                    if (gr < rows && gk < K) {
                        reg[u * 4 + i] = *reinterpret_cast<const uint4*>(X + gk * ld + gr);
                    } else {
                        reg[u * 4 + i] = make_uint4(0, 0, 0, 0);
                    }
                }
            }
        }
    }

    __device__ __forceinline__ void store(S* lds) const {
        const int tid = threadIdx.x;
        if constexpr (KROWS) {
#pragma unroll
            for (int i = 0; i < kLoads; ++i) {
                const int v = tid + i * THREADS;
                const int k = v / (R / V), c = v % (R / V);
                *reinterpret_cast<uint4*>(lds + k * KR_STRIDE + c * V) = reg[i];
            }
        } else if constexpr (KMAJOR) {
#pragma unroll
            for (int i = 0; i < kLoads; ++i) {
                const int v = tid + i * THREADS;
                const int r = v / (BK / V), kc = v % (BK / V);
                *reinterpret_cast<uint4*>(lds + r * LDS_STRIDE + kc * V) = reg[i];
            }
        } else {
            // Consecutive lanes take consecutive K blocks of one M/N block, so
            // the rows they write lie side by side in the LDS banks (with the
            // M/N block varying fastest, 32 lanes would land on two banks).
#pragma unroll
            for (int u = 0; u < kUnits; ++u) {
                const int unit = tid + u * THREADS;
                const int kb = unit % (BK / 4), rb = unit / (BK / 4);
                const uint4* in = reg + u * 4;
                if constexpr (sizeof(S) == 4) {
                    // 4 (k) x 4 (r) floats -> 4 rows of 4 consecutive k.
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const uint4 out = make_uint4(component(in[0], j), component(in[1], j),
                                                     component(in[2], j), component(in[3], j));
                        *reinterpret_cast<uint4*>(lds + (rb * V + j) * LDS_STRIDE + kb * 4) = out;
                    }
                } else {
                    // 4 (k) x 8 (r) 16-bit values -> 8 rows of 4 consecutive k.
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const int p = j / 2, hi = j % 2;
                        uint32_t w[4];
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const uint32_t c = component(in[i], p);
                            w[i] = hi ? (c >> 16) : (c & 0xffffu);
                        }
                        uint2 out;
                        out.x = w[0] | (w[1] << 16);
                        out.y = w[2] | (w[3] << 16);
                        *reinterpret_cast<uint2*>(lds + (rb * V + j) * LDS_STRIDE + kb * 4) = out;
                    }
                }
            }
        }
    }
};

// XCD-aware, L2-grouped tile order: consecutive ids land on the same XCD
// (blocks are dealt round-robin over the 8 XCDs), and each XCD walks its
// range in groups of kGroupM tile rows.
__device__ __forceinline__ void tile_coords(int bid, int grid_m, int grid_n, int& pm, int& pn) {
    const int total = grid_m * grid_n;
    int pid = bid;
    if (total % 8 == 0) pid = (bid % 8) * (total / 8) + bid / 8;
    const int in_group = kGroupM * grid_n;
    const int group = pid / in_group;
    const int first_m = group * kGroupM;
    const int size_m = grid_m - first_m < kGroupM ? grid_m - first_m : kGroupM;
    pm = first_m + (pid % in_group) % size_m;
    pn = (pid % in_group) / size_m;
}

// F32OUT: C is float32 (split-K partials of a 16-bit product), written as
// alpha acc with no Cin.
template <typename T, bool A_KMAJOR, bool B_KMAJOR, int BM, int BN, int WM, int WN, bool F32OUT = false>
__global__ __launch_bounds__(WM * WN * kWave) void gemm_mfma_kernel(GemmArgs p) {
    using S = typename Elem<T>::storage;
    constexpr int THREADS = WM * WN * kWave;
    using LA = TileLoader<T, BM, A_KMAJOR, THREADS>;
    using LB = TileLoader<T, BN, B_KMAJOR, THREADS>;
    constexpr int BK = Mfma<T>::BK, KSUB = Mfma<T>::KSUB;
    constexpr int LDS_STRIDE = LA::LDS_STRIDE;
    constexpr int kWaveM = BM / WM, kWaveN = BN / WN;
    constexpr int TM = kWaveM / 32, TN = kWaveN / 32;
    constexpr int STAGE = (BM + BN) * LDS_STRIDE;  // elements per LDS stage
    __shared__ __attribute__((aligned(16))) S lds[2 * STAGE];

    const int grid_m = static_cast<int>((p.m + BM - 1) / BM);
    const int grid_n = static_cast<int>((p.n + BN - 1) / BN);
    int pm, pn;
    tile_coords(blockIdx.x, grid_m, grid_n, pm, pn);
    const int64_t m0 = static_cast<int64_t>(pm) * BM, n0 = static_cast<int64_t>(pn) * BN;
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int wm = wave / WN, wn = wave % WN;
    const int half = lane / 32, l32 = lane % 32;

    // One batch entry per blockIdx.z (the host launches batches of at most
    // 65535); a loop over the batch here would keep every address live
    // across it and spill.
    {
        const int64_t bi = blockIdx.z;
        // Split-K partials: batch entry bi is the slice k = bi k .. of the
        // product's k_total, the last one shorter when k does not divide it.
        const int64_t kk = F32OUT && p.k_total - bi * p.k < p.k ? p.k_total - bi * p.k : p.k;
        const int64_t nk = (kk + BK - 1) / BK;
        const S* A = static_cast<const S*>(p.a) + bi * p.stride_a;
        const S* B = static_cast<const S*>(p.b) + bi * p.stride_b;
        f32x16 acc[TM][TN];
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

        LA la;
        LB lb;
        // Prologue: K tile 0 into stage 0, K tile 1 in flight.
        la.load(A, p.lda, m0, p.m, 0, kk);
        lb.load(B, p.ldb, n0, p.n, 0, kk);
        la.store(lds);
        lb.store(lds + BM * LDS_STRIDE);
        if (nk > 1) {
            la.load(A, p.lda, m0, p.m, BK, kk);
            lb.load(B, p.ldb, n0, p.n, BK, kk);
        }
        __syncthreads();
        for (int64_t kt = 0; kt < nk; ++kt) {
            const S* As = lds + (kt & 1) * STAGE;
            const S* Bs = As + BM * LDS_STRIDE;
            // Fragments are double-buffered across the K substeps: the LDS
            // reads for substep s + 1 are issued before the MFMAs of s, so
            // their latency hides behind the matrix work.
            constexpr int NSUB = BK / KSUB;
            uint4 af[2][TM], bf[2][TN];
            // A lane's 4 consecutive k (k0 + j for component j) of row or
            // column `rc`, from either LDS layout.
            auto frag = [&](const S* base, int rc, int k0, auto krows) -> uint4 {
                if constexpr (decltype(krows)::value) {
                    constexpr int KS = LA::KR_STRIDE;
                    static_assert(KS == LB::KR_STRIDE, "float32 tiles of one width");
                    const S* q = base + k0 * KS + rc;
                    uint4 v;
                    __builtin_memcpy(&v.x, q, 4);
                    __builtin_memcpy(&v.y, q + KS, 4);
                    __builtin_memcpy(&v.z, q + 2 * KS, 4);
                    __builtin_memcpy(&v.w, q + 3 * KS, 4);
                    return v;
                } else {
                    return *reinterpret_cast<const uint4*>(base + rc * LDS_STRIDE + k0);
                }
            };
            auto fetch = [&](int s, int buf) {
                const int k0 = s * KSUB + half * (KSUB / 2);
#pragma unroll
                for (int i = 0; i < TM; ++i)
                    af[buf][i] = frag(As, wm * kWaveM + i * 32 + l32, k0, std::integral_constant<bool, LA::KROWS>{});
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    bf[buf][j] = frag(Bs, wn * kWaveN + j * 32 + l32, k0, std::integral_constant<bool, LB::KROWS>{});
            };
            fetch(0, 0);
#pragma unroll
            for (int s = 0; s < NSUB; ++s) {
                if (s + 1 < NSUB) fetch(s + 1, (s + 1) & 1);
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        acc[i][j] = Mfma<T>::mma(af[s & 1][i], bf[s & 1][j], acc[i][j]);
            }
            // The other stage was last read in step kt - 1, before the
            // barrier that ended it: fill it with K tile kt + 1 and start
            // loading tile kt + 2.
            if (kt + 1 < nk) {
                S* next = lds + ((kt + 1) & 1) * STAGE;
                la.store(next);
                lb.store(next + BM * LDS_STRIDE);
            }
            if (kt + 2 < nk) {
                la.load(A, p.lda, m0, p.m, (kt + 2) * BK, kk);
                lb.load(B, p.ldb, n0, p.n, (kt + 2) * BK, kk);
            }
            __syncthreads();
        }

        // Epilogue: lane holds column l32 of each 32 x 32 tile, rows
        // 8 * (e / 4) + 4 * half + e % 4 for accumulator element e.
        if constexpr (F32OUT) {
            float* C = static_cast<float*>(p.c) + bi * p.stride_c;
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    const int64_t col = n0 + wn * kWaveN + j * 32 + l32;
                    const int64_t rbase = m0 + wm * kWaveM + i * 32 + 4 * half;
                    if (col >= p.n) continue;
#pragma unroll
                    for (int g = 0; g < 4; ++g)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int64_t row = rbase + 8 * g + r;
                            if (row < p.m) C[row * p.ldc + col] = p.alpha * acc[i][j][4 * g + r];
                        }
                }
            return;
        }
        S* C = static_cast<S*>(p.c) + bi * p.stride_c;
        const S* Cin = static_cast<const S*>(p.cin);
        if (p.trans_c) {
            // C^T: a lane's four consecutive rows r..r+3 of column `col` are
            // four consecutive elements of row `col` of the stored C, one
            // store when they are all inside and 16-byte aligned.  A store
            // instruction then covers 32 rows of C with 32 bytes each, and
            // the four of a row group complete each 128-byte line: these
            // stores keep the default cache policy, so L2 joins the pieces
            // before they reach HBM (float32 4096^3 as C^T: 1077 us, against
            // 1118 us with non-temporal stores, which reach memory as
            // partial lines).
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    const int64_t col = n0 + wn * kWaveN + j * 32 + l32;
                    const int64_t rbase = m0 + wm * kWaveM + i * 32 + 4 * half;
                    if (col >= p.n) continue;
                    S* cp = C + col * p.ldc + rbase;
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        float v[4];
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const float a = p.alpha * acc[i][j][4 * g + r];
                            const int64_t row = rbase + 8 * g + r;
                            if (p.beta == 0.0f || row >= p.m) {
                                v[r] = a;  // rows past M are not stored
                            } else {
                                const float c = Elem<T>::load(Cin[bi * p.cin_stride_b + row * p.cin_rs + col * p.cin_cs]);
                                v[r] = fmaf(p.beta, c, a);
                            }
                        }
                        S* dst = cp + 8 * g;
                        if constexpr (sizeof(S) == 4) {
                            if (rbase + 8 * g + 3 < p.m && (reinterpret_cast<uintptr_t>(dst) & 15u) == 0) {
                                *reinterpret_cast<uint4*>(dst) = make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]),
                                                                            __float_as_uint(v[2]), __float_as_uint(v[3]));
                                continue;
                            }
                        }
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            if (rbase + 8 * g + r < p.m) dst[r] = Elem<T>::store(v[r]);
                        }
                    }
                }
            return;
        }
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int64_t col = n0 + wn * kWaveN + j * 32 + l32;
                const int64_t rbase = m0 + wm * kWaveM + i * 32 + 4 * half;
                if (col >= p.n) continue;
                S* cp = C + rbase * p.ldc + col;
                if (p.beta == 0.0f) {
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            if (rbase + 8 * g + r < p.m) {
                                put_c(&cp[r * p.ldc], Elem<T>::store(p.alpha * acc[i][j][4 * g + r]));
                            }
                        }
                        cp += 8 * p.ldc;
                    }
                } else if (p.cin_rs == 0) {
                    // A bias along N (addmm / linear): one value per column.
                    const float c = p.beta * Elem<T>::load(Cin[bi * p.cin_stride_b + col * p.cin_cs]);
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            if (rbase + 8 * g + r < p.m) {
                                put_c(&cp[r * p.ldc], Elem<T>::store(fmaf(p.alpha, acc[i][j][4 * g + r], c)));
                            }
                        }
                        cp += 8 * p.ldc;
                    }
                } else {
                    const S* ci = Cin + bi * p.cin_stride_b + rbase * p.cin_rs + col * p.cin_cs;
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            if (rbase + 8 * g + r < p.m) {
                                const float c = Elem<T>::load(ci[r * p.cin_rs]);
                                put_c(&cp[r * p.ldc],
                                      Elem<T>::store(fmaf(p.beta, c, p.alpha * acc[i][j][4 * g + r])));
                            }
                        }
                        cp += 8 * p.ldc;
                        ci += 8 * p.cin_rs;
                    }
                }
            }
    }
}

namespace big {

// 256 x 256 x 64 tiles over WM x WN waves (2 x 2 waves of 128 x 128, or
// 2 x 4 of 128 x 64), every tile full.
//
// Operand tiles move from memory straight into LDS with buffer loads (16
// bytes a lane, no registers in between).  Each operand tile is 32 KB in one
// of two layouts, swizzled for gfx950's LDS of 64 four-byte banks (256 bytes
// a clock); both read at zero SQ_LDS_BANK_CONFLICT in every layout, which is
// what settles a swizzle here (the reasoning below, 16 lanes of a
// ds_read_b128 and 32 of an 8-byte read a clock, explains these two but is
// not a complete model of the hardware):
//   * K-major operand: 256 rows (M or N) of 128 bytes, one row = the tile's
//     64 k; logical 16-byte chunk c of row r sits at slot c ^ kswz(r).  A
//     load instruction fills 8 rows; a fragment read (ds_read_b128: 32 rows,
//     one chunk) puts each 16-lane group's 16 rows on 64 distinct banks.
//   * M/N-major operand (a transposed view, read in place): 64 rows (k) of
//     512 bytes, chunk c of row k at slot c ^ nswz(k).  A load instruction
//     fills 2 rows.  Fragments come from ds_read_b64_tr_b16, which hands
//     each lane of a 16-lane group one column of a 4 x 16 block: two of them
//     give a lane its 8 consecutive k; the 4 rows x 64 bytes that 32 lanes
//     read fall on 64 distinct banks.
// Both swizzles also keep 8 lanes of a b128 read (16 of a b64 read) on 32
// distinct banks.
// The loads for K tile kt + 1 go out during the first half of step kt into
// the other LDS stage, spread between the MFMAs.
constexpr int BM = 256, BN = 256, BK = 64;
constexpr int TILE = 256 * 128;   // bytes per operand tile
constexpr int STAGE = 2 * TILE;   // bytes per LDS stage
typedef __attribute__((address_space(3))) void* lds_ptr;
typedef short short4_t __attribute__((ext_vector_type(4)));

// K-major: rows r and r + 8 (one 16-lane group) differ in the low bit of the
// slot; rows of one parity (the same half of a 256-byte bank line) take 8
// distinct slots.
__device__ __forceinline__ int kswz(int r) { return (r & 7) ^ ((r >> 3) & 1); }
// M/N-major: rows k..k+3 move a 4-chunk span (64 bytes) to four distinct
// quarters of a bank line, and a 2-chunk span to four distinct slots mod 8.
__device__ __forceinline__ int nswz(int k) { return (2 * (k & 3)) ^ (8 * (k & 1)); }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), bytes,
                                             0x00020000);
}

// One operand: the block's 256-wide panel of X (M or N from mn0), loaded by
// W waves, read as T 32-wide tiles per wave.
template <bool KMAJOR, int W, int T>
struct Operand {
    static constexpr int kIssue = 32 / W;  // load instructions per wave per K tile
    __amdgpu_buffer_rsrc_t res;
    uint32_t voff, sbase, sstep, kstep;
    int frag[4];       // per-lane fragment byte offsets (K-major: per substep; M/N-major: per tile)

    __device__ __forceinline__ void init(const void* X, int64_t ld, int64_t mn0, int64_t K, int wave,
                                         int lane, int wbase) {
        const int l32 = lane % 32, half = lane / 32;
        if constexpr (KMAJOR) {
            // element (r, k) at X[r * ld + k]; a load's lane L fills slot L % 8
            // of row L / 8 of its 8-row group
            res = rsrc(static_cast<const uint16_t*>(X) + mn0 * ld, static_cast<uint32_t>(256 * ld * 2));
            const int row = lane >> 3, chunk = (lane & 7) ^ kswz(8 * wave + row);
            voff = static_cast<uint32_t>((row * ld + chunk * 8) * 2);
            sbase = static_cast<uint32_t>(wave * 8 * ld * 2);
            sstep = static_cast<uint32_t>(W * 8 * ld * 2);
            kstep = BK * 2;
#pragma unroll
            for (int s = 0; s < 4; ++s)
                frag[s] = (wbase + l32) * 128 + (((2 * s + half) ^ kswz(l32)) << 4);
        } else {
            // element (k, r) at X[k * ld + r]; a load fills 2 rows of k
            res = rsrc(static_cast<const uint16_t*>(X) + mn0, static_cast<uint32_t>(K * ld * 2));
            const int row = lane >> 5;
            const int chunk = (lane & 31) ^ nswz(2 * (wave & 1) + row);
            voff = static_cast<uint32_t>((row * ld + chunk * 8) * 2);
            sbase = static_cast<uint32_t>(2 * wave * ld * 2);
            sstep = static_cast<uint32_t>(2 * W * ld * 2);
            kstep = static_cast<uint32_t>(BK * ld * 2);
            // Transposed reads: lane p of 16-lane group g addresses row
            // 8 * half + p / 4 (+ 16 s + 4 h) and column 16 (g & 1) + 4 (p % 4)
            // of the wave's 32-wide tile t.
            const int g = lane / 16, pl = lane % 16;
            const int krow = 8 * half + pl / 4;
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const int col = wbase + t * 32 + 16 * (g & 1) + 4 * (pl % 4);
                frag[t] = krow * 512 + (((col / 8) ^ nswz(krow)) << 4) + (col % 8) * 2;
            }
        }
    }

    // Loads of K tile kt into `tile` (this wave's share of the 32 instructions).
    __device__ __forceinline__ void issue(int kt, char* tile, int wave) const {
        const uint32_t kb = static_cast<uint32_t>(kt) * kstep;
#pragma unroll
        for (int i = 0; i < kIssue; ++i) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(res, (lds_ptr)(tile + (i * W + wave) * 1024), 16, voff,
                                                     sbase + i * sstep + kb, 0, 0);
        }
    }

    // The 8 k of substep s for the wave's 32-wide tile t.
    __device__ __forceinline__ uint4 read(const char* tile, int t, int s) const {
        if constexpr (KMAJOR) {
            return *reinterpret_cast<const uint4*>(tile + t * 32 * 128 + frag[s]);
        } else {
            const char* q = tile + frag[t] + s * 16 * 512;
            const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4_t*)(q));
            const short4_t hi =
                __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4_t*)(q + 4 * 512));
            uint4 v;
            __builtin_memcpy(&v, &lo, 8);
            __builtin_memcpy(reinterpret_cast<char*>(&v) + 8, &hi, 8);
            return v;
        }
    }
};

// MF MFMAs with RD LDS reads and LD loads spread evenly between them.
template <int MF, int RD, int LD, int Q>
__device__ __forceinline__ void interleave_slot() {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    constexpr int r = RD * (Q + 1) / MF - RD * Q / MF;
    constexpr int l = LD * (Q + 1) / MF - LD * Q / MF;
    if constexpr (r > 0) __builtin_amdgcn_sched_group_barrier(0x100, r, 0);
    if constexpr (l > 0) __builtin_amdgcn_sched_group_barrier(0x020, l, 0);
}
template <int MF, int RD, int LD, int... Q>
__device__ __forceinline__ void interleave_slots(std::integer_sequence<int, Q...>) {
    (interleave_slot<MF, RD, LD, Q>(), ...);
}
template <int MF, int RD, int LD>
__device__ __forceinline__ void interleave() {
    interleave_slots<MF, RD, LD>(std::make_integer_sequence<int, MF>{});
}

template <typename T, bool A_KMAJOR, bool B_KMAJOR, int WM, int WN>
__global__ __launch_bounds__(WM * WN * kWave, (WM * WN) / 4) void gemm_big_kernel(GemmArgs p) {
    using S = typename Elem<T>::storage;
    static_assert(sizeof(S) == 2, "16-bit operands");
    constexpr int W = WM * WN;
    constexpr int TM = BM / WM / 32, TN = BN / WN / 32;
    // Two LDS objects rather than one array: the compiler can then tell that
    // the loads filling one stage do not touch the stage being read, and
    // leaves them in flight across the step.
    __shared__ __attribute__((aligned(1024))) char lds0[STAGE];
    __shared__ __attribute__((aligned(1024))) char lds1[STAGE];

    const int grid_m = static_cast<int>(p.m / BM), grid_n = static_cast<int>(p.n / BN);
    int pm, pn;
    tile_coords(blockIdx.x, grid_m, grid_n, pm, pn);
    const int64_t m0 = static_cast<int64_t>(pm) * BM, n0 = static_cast<int64_t>(pn) * BN;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = threadIdx.x % kWave;
    const int wm = wave / WN, wn = wave % WN;
    const int l32 = lane % 32, half = lane / 32;
    const int nk = static_cast<int>(p.k / BK);
    const int64_t bi = blockIdx.z;

    Operand<A_KMAJOR, W, TM> oa;
    Operand<B_KMAJOR, W, TN> ob;
    oa.init(static_cast<const S*>(p.a) + bi * p.stride_a, p.lda, m0, p.k, wave, lane, wm * TM * 32);
    ob.init(static_cast<const S*>(p.b) + bi * p.stride_b, p.ldb, n0, p.k, wave, lane, wn * TN * 32);

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    uint4 af[2][TM], bf[2][TN];
    auto fetch = [&](const char* stage, int s, int buf) {
#pragma unroll
        for (int i = 0; i < TM; ++i) af[buf][i] = oa.read(stage, i, s);
#pragma unroll
        for (int j = 0; j < TN; ++j) bf[buf][j] = ob.read(stage + TILE, j, s);
    };
    auto mma = [&](int buf) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) acc[i][j] = Mfma<T>::mma(af[buf][i], bf[buf][j], acc[i][j]);
    };
    // Per substep: TM x TN MFMAs, and a b128 fragment read per K-major tile
    // or two transposed b64 reads per M/N-major one.
    constexpr int kMf = TM * TN;
    constexpr int kReads = TM * (A_KMAJOR ? 1 : 2) + TN * (B_KMAJOR ? 1 : 2);
    // One K step out of `cur`, entered with substep 0's fragments in
    // flight.  Substeps 0-2 each run their MFMAs interleaved with the next
    // substep's fragment reads (and, in substep 0, this wave's loads of B
    // for the next K tile).  The step then waits for its loads and the
    // barrier, and starts reading the next step's first fragments before
    // running substep 3's MFMAs, whose operands are in registers.  After
    // that barrier no wave reads `cur` again, so substep 3 also issues the
    // loads of A for the K tile after next into it: A's loads get four
    // substeps to land and B's three, against three and two when both went
    // out in substeps 0 and 1 (bf16 linear 8192 x 4096 x 11008 733 -> 706 us
    // on average over three alternating runs, 4096^3 1-2 % faster, the same
    // bits).
    // do_issue: load B of K tile kt_next into `next`; issue_a: load A of
    // K tile kt_next + 1 into `cur` after the barrier.
    auto body = [&](char* cur, char* next, int kt_next, auto do_issue, auto has_next, auto issue_a) {
        constexpr bool kIssue = decltype(do_issue)::value;
        constexpr bool kIssueA = decltype(issue_a)::value;
#pragma unroll
        for (int s = 0; s < 3; ++s) {
            fetch(cur, s + 1, (s + 1) & 1);
            if constexpr (kIssue) {
                if (s == 0) ob.issue(kt_next, next + TILE, wave);
            }
            mma(s & 1);
            if (kIssue && s == 0) {
                interleave<kMf, kReads, 32 / W>();
            } else {
                interleave<kMf, kReads, 0>();
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (decltype(has_next)::value) {
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            fetch(next, 0, 0);
            if constexpr (kIssueA) oa.issue(kt_next + 1, cur, wave);
            mma(1);
            interleave<kMf, kReads, kIssueA ? 32 / W : 0>();
        } else {
            mma(1);
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    // K tile 0 whole, and A of K tile 1 (the host guarantees nk >= 2).
    oa.issue(0, lds0, wave);
    ob.issue(0, lds0 + TILE, wave);
    oa.issue(1, lds1, wave);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    fetch(lds0, 0, 0);
    // Steps in pairs (stage 0 then stage 1), so every access names its LDS
    // object statically; the host guarantees an even number of K tiles.
    // Inside the loop kt + 3 <= nk - 1, so A of K tile kt_next + 1 exists.
    for (int kt = 0; kt + 2 < nk; kt += 2) {
        body(lds0, lds1, kt + 1, std::true_type{}, std::true_type{}, std::true_type{});
        body(lds1, lds0, kt + 2, std::true_type{}, std::true_type{}, std::true_type{});
    }
    body(lds0, lds1, nk - 1, std::true_type{}, std::true_type{}, std::false_type{});
    body(lds1, lds0, 0, std::false_type{}, std::false_type{}, std::false_type{});

    // Epilogue: lane holds column l32 of each 32 x 32 tile, rows
    // 8 * (e / 4) + 4 * half + e % 4 for accumulator element e.
    S* C = static_cast<S*>(p.c) + bi * p.stride_c;
    const S* Cin = static_cast<const S*>(p.cin);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int64_t col = n0 + wn * TN * 32 + j * 32 + l32;
            const int64_t rbase = m0 + wm * TM * 32 + i * 32 + 4 * half;
            S* cp = C + rbase * p.ldc + col;
            if (p.beta == 0.0f) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) put_c(&cp[r * p.ldc], Elem<T>::store(p.alpha * acc[i][j][4 * g + r]));
                    cp += 8 * p.ldc;
                }
            } else if (p.cin_rs == 0) {
                const float c = p.beta * Elem<T>::load(Cin[bi * p.cin_stride_b + col * p.cin_cs]);
#pragma unroll
                for (int g = 0; g < 4; ++g) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) put_c(&cp[r * p.ldc], Elem<T>::store(fmaf(p.alpha, acc[i][j][4 * g + r], c)));
                    cp += 8 * p.ldc;
                }
            } else {
                const S* ci = Cin + bi * p.cin_stride_b + rbase * p.cin_rs + col * p.cin_cs;
#pragma unroll
                for (int g = 0; g < 4; ++g) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float c = Elem<T>::load(ci[r * p.cin_rs]);
                        put_c(&cp[r * p.ldc], Elem<T>::store(fmaf(p.beta, c, p.alpha * acc[i][j][4 * g + r])));
                    }
                    cp += 8 * p.ldc;
                    ci += 8 * p.cin_rs;
                }
            }
        }
}

template <typename T>
bool eligible(const GemmArgs& p, int cus) {
    const bool a_kmajor = !p.trans_a, b_kmajor = p.trans_b;
    // A block addresses its panel through one buffer resource: 256 rows of
    // ld (K-major, needs ld >= K) or K rows of ld (M/N-major, needs
    // ld >= 256), under 4 GiB.
    auto panel_ok = [&](const void* x, int64_t ld, int64_t stride, bool kmajor) {
        const int64_t bytes = kmajor ? 256 * ld * 2 : p.k * ld * 2;
        return aligned16(x) && ld % 8 == 0 && stride % 8 == 0 && bytes < (int64_t(1) << 32) &&
               (kmajor ? ld >= p.k : ld >= 256);
    };
    return p.m % BM == 0 && p.n % BN == 0 && p.k % (2 * BK) == 0 &&
           panel_ok(p.a, p.lda, p.stride_a, a_kmajor) && panel_ok(p.b, p.ldb, p.stride_b, b_kmajor) &&
           (p.m / BM) * (p.n / BN) * p.batch >= cus && (p.m / BM) * (p.n / BN) < (int64_t(1) << 31);
}

template <typename T, int WM, int WN>
void launch_shape(const GemmArgs& whole, hipStream_t stream) {
    constexpr int64_t kMaxZ = 65535;
    using S = typename Elem<T>::storage;
    const bool a_kmajor = !whole.trans_a, b_kmajor = whole.trans_b;
    for (int64_t b0 = 0; b0 < whole.batch; b0 += kMaxZ) {
        GemmArgs p = whole;
        p.batch = whole.batch - b0 < kMaxZ ? whole.batch - b0 : kMaxZ;
        p.a = static_cast<const S*>(whole.a) + b0 * whole.stride_a;
        p.b = static_cast<const S*>(whole.b) + b0 * whole.stride_b;
        p.c = static_cast<S*>(whole.c) + b0 * whole.stride_c;
        if (whole.cin != nullptr) p.cin = static_cast<const S*>(whole.cin) + b0 * whole.cin_stride_b;
        const dim3 grid(static_cast<unsigned>((p.m / BM) * (p.n / BN)), 1u, static_cast<unsigned>(p.batch));
        constexpr int THREADS = WM * WN * kWave;
        if (a_kmajor && b_kmajor) {
            gemm_big_kernel<T, true, true, WM, WN><<<grid, THREADS, 0, stream>>>(p);
        } else if (a_kmajor) {
            gemm_big_kernel<T, true, false, WM, WN><<<grid, THREADS, 0, stream>>>(p);
        } else if (b_kmajor) {
            gemm_big_kernel<T, false, true, WM, WN><<<grid, THREADS, 0, stream>>>(p);
        } else {
            gemm_big_kernel<T, false, false, WM, WN><<<grid, THREADS, 0, stream>>>(p);
        }
        TP_AMD_HIP_CHECK(hipGetLastError());
    }
}

// Four waves of 128 x 128 for long K.  With K <= 256 (two to four K steps:
// bmm of attention-sized products) the prologue and the epilogue dominate,
// and eight waves of 128 x 64 -- two per SIMD -- overlap them: bf16
// 64 x 512 x 128 x 512 bmm 15.9 -> 13.5 us.  At 4096^3 the two shapes
// measure the same.
template <typename T>
void launch(const GemmArgs& p, hipStream_t stream) {
    if (p.k <= 256) {
        launch_shape<T, 2, 4>(p, stream);
    } else {
        launch_shape<T, 2, 2>(p, stream);
    }
}

}  // namespace big

// Short products (16-bit, K = 64 or 128: attention-sized bmm) are bound by
// storing C, not by the MFMAs: bf16 64 x 512 x 128 x 512 reads 16 MB and
// writes 32 MB.  Here all of K goes into LDS at once (one or two of the big
// kernel's stages, same layouts), one barrier, and each of the 8 waves then
// works through its 128 x 64 patch one 32 x 32 tile at a time -- the tile's
// MFMAs over all of K, then its stores -- so the stores of one tile drain
// while the MFMAs of the next run, instead of all of C going out after all
// the products.  The grid is one dimension over batch x tiles, numbered so a
// batch's tiles (which share A and B panels) stay on one XCD and its L2.
// Measured on the config-5a bmm against the big kernel on the same box:
// 12.5 against 15.6 us (rocprof), hipBLASLt 15.0 us.
namespace smallk {

constexpr int W = 8, WN = 4, TM = 4, TN = 2;

template <typename T, bool A_KMAJOR, bool B_KMAJOR>
__global__ __launch_bounds__(W * kWave, 1) void gemm_smallk_kernel(GemmArgs p) {
    using S = typename Elem<T>::storage;
    using big::BK;
    using big::STAGE;
    using big::TILE;
    __shared__ __attribute__((aligned(1024))) char lds0[STAGE];
    __shared__ __attribute__((aligned(1024))) char lds1[STAGE];
    const int grid_n = static_cast<int>(p.n / big::BN);
    const int tiles = static_cast<int>(p.m / big::BM) * grid_n;
    const int total = static_cast<int>(gridDim.x);
    const int pid = total % 8 == 0 ? (blockIdx.x % 8) * (total / 8) + blockIdx.x / 8 : blockIdx.x;
    const int64_t bi = pid / tiles;
    const int tile = pid % tiles;
    const int64_t m0 = static_cast<int64_t>(tile / grid_n) * big::BM;
    const int64_t n0 = static_cast<int64_t>(tile % grid_n) * big::BN;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = threadIdx.x % kWave;
    const int wm = wave / WN, wn = wave % WN;
    const int l32 = lane % 32, half = lane / 32;
    const int nk = static_cast<int>(p.k / BK);
    big::Operand<A_KMAJOR, W, TM> oa;
    big::Operand<B_KMAJOR, W, TN> ob;
    oa.init(static_cast<const S*>(p.a) + bi * p.stride_a, p.lda, m0, p.k, wave, lane, wm * TM * 32);
    ob.init(static_cast<const S*>(p.b) + bi * p.stride_b, p.ldb, n0, p.k, wave, lane, wn * TN * 32);
    oa.issue(0, lds0, wave);
    ob.issue(0, lds0 + TILE, wave);
    if (nk > 1) {
        oa.issue(1, lds1, wave);
        ob.issue(1, lds1 + TILE, wave);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    S* C = static_cast<S*>(p.c) + bi * p.stride_c;
    const S* Cin = static_cast<const S*>(p.cin);
    // Tiles in a fixed order, fully unrolled, so every fragment offset is
    // static; the scheduling barrier keeps the next tile's reads out of this
    // one's stores (otherwise the registers run out and spill).
#pragma unroll
    for (int t = 0; t < TM * TN; ++t) {
        __builtin_amdgcn_sched_barrier(0);
        const int i = t % TM, j = t / TM;
        f32x16 acc;
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
        for (int kt = 0; kt < nk; ++kt) {
            const char* st = kt == 0 ? lds0 : lds1;
#pragma unroll
            for (int s = 0; s < 4; ++s) acc = Mfma<T>::mma(oa.read(st, i, s), ob.read(st + TILE, j, s), acc);
        }
        const int64_t col = n0 + wn * TN * 32 + j * 32 + l32;
        const int64_t rbase = m0 + wm * TM * 32 + i * 32 + 4 * half;
        S* cp = C + rbase * p.ldc + col;
        if (p.beta == 0.0f) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
#pragma unroll
                for (int r = 0; r < 4; ++r) put_c(&cp[r * p.ldc], Elem<T>::store(p.alpha * acc[4 * g + r]));
                cp += 8 * p.ldc;
            }
        } else if (p.cin_rs == 0) {
            const float c = p.beta * Elem<T>::load(Cin[bi * p.cin_stride_b + col * p.cin_cs]);
#pragma unroll
            for (int g = 0; g < 4; ++g) {
#pragma unroll
                for (int r = 0; r < 4; ++r) put_c(&cp[r * p.ldc], Elem<T>::store(fmaf(p.alpha, acc[4 * g + r], c)));
                cp += 8 * p.ldc;
            }
        } else {
            const S* ci = Cin + bi * p.cin_stride_b + rbase * p.cin_rs + col * p.cin_cs;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float c = Elem<T>::load(ci[r * p.cin_rs]);
                    put_c(&cp[r * p.ldc], Elem<T>::store(fmaf(p.beta, c, p.alpha * acc[4 * g + r])));
                }
                cp += 8 * p.ldc;
                ci += 8 * p.cin_rs;
            }
        }
    }
}

// K of one or two 64-deep stages, full 256 x 256 tiles, the big kernel's
// panel rules, and enough tiles to give every CU one.
template <typename T>
bool eligible(const GemmArgs& p, int cus) {
    const bool a_kmajor = !p.trans_a, b_kmajor = p.trans_b;
    auto panel_ok = [&](const void* x, int64_t ld, int64_t stride, bool kmajor) {
        const int64_t bytes = kmajor ? 256 * ld * 2 : p.k * ld * 2;
        return aligned16(x) && ld % 8 == 0 && stride % 8 == 0 && bytes < (int64_t(1) << 32) &&
               (kmajor ? ld >= p.k : ld >= 256);
    };
    const int64_t tiles = (p.m / big::BM) * (p.n / big::BN) * p.batch;
    return (p.k == 64 || p.k == 128) && p.m % big::BM == 0 && p.n % big::BN == 0 &&
           panel_ok(p.a, p.lda, p.stride_a, a_kmajor) && panel_ok(p.b, p.ldb, p.stride_b, b_kmajor) &&
           tiles >= cus && tiles < (int64_t(1) << 31);
}

template <typename T>
void launch(const GemmArgs& p, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>((p.m / big::BM) * (p.n / big::BN) * p.batch));
    const bool a_kmajor = !p.trans_a, b_kmajor = p.trans_b;
    if (a_kmajor && b_kmajor) {
        gemm_smallk_kernel<T, true, true><<<grid, W * kWave, 0, stream>>>(p);
    } else if (a_kmajor) {
        gemm_smallk_kernel<T, true, false><<<grid, W * kWave, 0, stream>>>(p);
    } else if (b_kmajor) {
        gemm_smallk_kernel<T, false, true><<<grid, W * kWave, 0, stream>>>(p);
    } else {
        gemm_smallk_kernel<T, false, false><<<grid, W * kWave, 0, stream>>>(p);
    }
    TP_AMD_HIP_CHECK(hipGetLastError());
}

}  // namespace smallk

// An operand the matrix-core kernels read in place: 16-byte aligned, and its
// leading dimension, batch stride and contiguous extent (K when K-major, M or
// N otherwise) whole numbers of V-element packets.
template <typename T>
bool operand_ok(const void* ptr, int64_t ld, int64_t stride, bool kmajor, int64_t mn, int64_t k) {
    constexpr int V = Mfma<T>::V;
    return aligned16(ptr) && ld % V == 0 && stride % V == 0 && (kmajor ? k : mn) % V == 0;
}

bool tiles_fit(const GemmArgs& p) {
    return (p.m + 127) / 128 * ((p.n + 127) / 128) < (int64_t(1) << 31);
}

template <typename T>
bool mfma_eligible(const GemmArgs& p) {
    return p.k > 0 && operand_ok<T>(p.a, p.lda, p.stride_a, !p.trans_a, p.m, p.k) &&
           operand_ok<T>(p.b, p.ldb, p.stride_b, p.trans_b, p.n, p.k) && tiles_fit(p);
}

template <typename T, int BM, int BN, int WM, int WN, bool F32OUT = false>
void launch_chunk(const GemmArgs& p, hipStream_t stream) {
    constexpr int THREADS = WM * WN * kWave;
    const int64_t tiles = ((p.m + BM - 1) / BM) * ((p.n + BN - 1) / BN);
    const dim3 grid(static_cast<unsigned>(tiles), 1u, static_cast<unsigned>(p.batch));
    const bool a_kmajor = !p.trans_a, b_kmajor = p.trans_b;
    if (a_kmajor && b_kmajor) {
        gemm_mfma_kernel<T, true, true, BM, BN, WM, WN, F32OUT><<<grid, THREADS, 0, stream>>>(p);
    } else if (a_kmajor) {
        gemm_mfma_kernel<T, true, false, BM, BN, WM, WN, F32OUT><<<grid, THREADS, 0, stream>>>(p);
    } else if (b_kmajor) {
        gemm_mfma_kernel<T, false, true, BM, BN, WM, WN, F32OUT><<<grid, THREADS, 0, stream>>>(p);
    } else {
        gemm_mfma_kernel<T, false, false, BM, BN, WM, WN, F32OUT><<<grid, THREADS, 0, stream>>>(p);
    }
    TP_AMD_HIP_CHECK(hipGetLastError());
}

template <typename T, int BM, int BN, int WM, int WN, bool F32OUT = false>
void launch_config(const GemmArgs& whole, hipStream_t stream) {
    constexpr int64_t kMaxZ = 65535;
    using S = typename Elem<T>::storage;
    for (int64_t b0 = 0; b0 < whole.batch; b0 += kMaxZ) {
        GemmArgs p = whole;
        p.batch = whole.batch - b0 < kMaxZ ? whole.batch - b0 : kMaxZ;
        p.a = static_cast<const S*>(whole.a) + b0 * whole.stride_a;
        p.b = static_cast<const S*>(whole.b) + b0 * whole.stride_b;
        p.c = F32OUT ? static_cast<void*>(static_cast<float*>(whole.c) + b0 * whole.stride_c)
                     : static_cast<void*>(static_cast<S*>(whole.c) + b0 * whole.stride_c);
        if (whole.cin != nullptr) p.cin = static_cast<const S*>(whole.cin) + b0 * whole.cin_stride_b;
        if (F32OUT) p.k_total = whole.k_total - b0 * whole.k;
        launch_chunk<T, BM, BN, WM, WN, F32OUT>(p, stream);
    }
}
// Split K for float32 products with too few 128 x 128 tiles to fill the
// CUs: a single matrix whose K dwarfs M x N (mm 1024^3 has 64 tiles; the
// Linear(4096, 1024) of a 256-row batch has 16, each running K = 4096 alone
// on one CU).  S slices of K ride on the kernel's batch index and write
// float32 partial products into a workspace [S][M][N]; splitk_finish_kernel
// then adds the slices in slice order -- the result does not depend on
// timing -- and applies alpha, beta Cin and the epilogue's rounding.
// S doubles while the tiles times S still fit one block per CU and every
// slice keeps at least 128 of K, a multiple of the kernel's BK = 32.
constexpr int kFinishBlock = 256;

int splitk_slices(const GemmArgs& p, int cus, int tile = 128, int min_k = 128, int bk = 32) {
    if (p.batch != 1) return 1;
    const int64_t tiles = ((p.m + tile - 1) / tile) * ((p.n + tile - 1) / tile);
    int s = 1;
    while (tiles * s * 2 <= cus && p.k % (s * 2 * bk) == 0 && p.k / (s * 2) >= min_k) s *= 2;
    return s;
}

// Slice 0 + slice 1 + ... of element i, added in slice order; the loads go
// out four at a time ahead of their adds.
__device__ __forceinline__ float sum_slices(const float* part, int slices, int64_t mn, int64_t i) {
    float acc = part[i];
    int s = 1;
    for (; s + 4 <= slices; s += 4) {
        const float v0 = part[s * mn + i], v1 = part[(s + 1) * mn + i];
        const float v2 = part[(s + 2) * mn + i], v3 = part[(s + 3) * mn + i];
        acc += v0;
        acc += v1;
        acc += v2;
        acc += v3;
    }
    for (; s < slices; ++s) acc += part[s * mn + i];
    return acc;
}

// A float32 product of 33 to 64 rows (or columns) against a wide operand of
// at least 128 tiles of 64 (a small batch through a Linear of 8192 or more
// outputs): 64 x 64 tiles of two waves, K split up to four blocks a CU.
// The thin kernel leaves these here.  Measured (64 x 11008 x 4096, W
// rotated beyond the Infinity Cache): x W^T 91-95 against 104-114 us on
// the thin kernel, x W 94-102 against 106-140 us; with 4096 columns (64
// tiles) the thin kernel stays faster (101-110 against 109-114 us).
int splitk32_small_batch(const GemmArgs& p, int cus) {
    const int64_t thin = std::min(p.m, p.n), wide = std::max(p.m, p.n);
    if (p.batch != 1 || thin <= 32 || thin > 64 || (wide + 63) / 64 < 128) return 1;
    return splitk_slices(p, 4 * cus, 64);
}

// c = alpha * sum of the slices (+ beta Cin), the same expressions as the
// kernels' epilogue; one thread an element, consecutive threads along a row.
__global__ __launch_bounds__(kFinishBlock) void splitk_finish_kernel(const float* part, int slices, int64_t m,
                                                               int64_t n, float alpha, float beta,
                                                               const float* cin, int64_t cin_rs,
                                                               int64_t cin_cs, float* c, int64_t ldc) {
    const int64_t mn = m * n;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kFinishBlock + threadIdx.x; i < mn;
         i += static_cast<int64_t>(gridDim.x) * kFinishBlock) {
        const float acc = sum_slices(part, slices, mn, i);
        const int64_t r = i / n, col = i % n;
        float v;
        if (beta == 0.0f) {
            v = alpha * acc;
        } else if (cin_rs == 0) {
            v = fmaf(alpha, acc, beta * cin[col * cin_cs]);
        } else {
            v = fmaf(beta, cin[r * cin_rs + col * cin_cs], alpha * acc);
        }
        c[r * ldc + col] = v;
    }
}

template <int BM, int BN, int WM, int WN>
void launch_splitk(const GemmArgs& p, int slices, hipStream_t stream, int device) {
    const int64_t mn = p.m * p.n;
    Workspace ws(static_cast<size_t>(slices * mn) * sizeof(float), device);
    GemmArgs q = p;
    q.batch = slices;
    q.k = p.k / slices;
    q.stride_a = p.trans_a ? q.k * p.lda : q.k;  // slice s starts at k = s q.k
    q.stride_b = p.trans_b ? q.k : q.k * p.ldb;
    q.alpha = 1.0f;
    q.beta = 0.0f;
    q.cin = nullptr;
    q.c = ws.get();
    q.ldc = p.n;
    q.stride_c = mn;
    launch_config<float, BM, BN, WM, WN>(q, stream);
    const int64_t blocks = std::min<int64_t>((mn + kFinishBlock - 1) / kFinishBlock, 4 * int64_t{cu_count(device)});
    splitk_finish_kernel<<<static_cast<unsigned>(blocks), kFinishBlock, 0, stream>>>(
        static_cast<const float*>(ws.get()), slices, p.m, p.n, p.alpha, p.beta,
        static_cast<const float*>(p.cin), p.cin_rs, p.cin_cs, static_cast<float*>(p.c), p.ldc);
    TP_AMD_HIP_CHECK(hipGetLastError());
}

// The same split for 16-bit products: the slices write float32 partials
// (the tile kernel's F32OUT epilogue) and the finish adds them in slice
// order and rounds once to the output type.
template <typename T>
__global__ __launch_bounds__(kFinishBlock) void splitk_finish16_kernel(
    const float* part, int slices, int64_t m, int64_t n, float alpha, float beta,
    const typename Elem<T>::storage* cin, int64_t cin_rs, int64_t cin_cs, typename Elem<T>::storage* c,
    int64_t ldc) {
    const int64_t mn = m * n;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kFinishBlock + threadIdx.x; i < mn;
         i += static_cast<int64_t>(gridDim.x) * kFinishBlock) {
        const float acc = sum_slices(part, slices, mn, i);
        const int64_t r = i / n, col = i % n;
        float v;
        if (beta == 0.0f) {
            v = alpha * acc;
        } else if (cin_rs == 0) {
            v = fmaf(alpha, acc, beta * Elem<T>::load(cin[col * cin_cs]));
        } else {
            v = fmaf(beta, Elem<T>::load(cin[r * cin_rs + col * cin_cs]), alpha * acc);
        }
        c[r * ldc + col] = Elem<T>::store(v);
    }
}

// The 16-bit split: the most slices that keep the 128 x 128 tiles times
// the slices within two blocks a CU, with slices of a multiple of BK and at
// least kSplit16MinK; the last slice is shorter when K is not a multiple of
// the slice.  A product of one row of tiles (a small batch, min(M, N) <=
// 128) takes slices of kSplit16ShortK when that still gives every CU a
// block: bf16 17-64 x 11008 x 4096 26-32 us against 29-34 us, 128 x 4096
// x 4096 22.4 against 24.5 us (W rotated beyond the Infinity Cache).  With
// more rows of tiles the extra partials cost more than the blocks gain
// (256 x 4096 x 4096 30.9 against 29.1 us), and 1024^3 in slices of 512
// ran 19.5 against 13.5 us unsplit.
struct SplitPlan {
    int64_t slices = 1, ks = 0;
};

constexpr int64_t kSplit16MinK = 1024;
constexpr int64_t kSplit16ShortK = 512;

SplitPlan splitk16_slices(const GemmArgs& p, int64_t max_blocks, int64_t min_k, int64_t bk) {
    SplitPlan plan;
    if (p.batch != 1) return plan;
    const int64_t tiles = ((p.m + 127) / 128) * ((p.n + 127) / 128);
    for (int64_t s = max_blocks / tiles; s > 1; --s) {
        const int64_t ks = ((p.k + s - 1) / s + bk - 1) / bk * bk;
        if (ks < min_k) continue;
        plan.ks = ks;
        plan.slices = (p.k + ks - 1) / ks;
        break;
    }
    return plan;
}

SplitPlan splitk16_plan(const GemmArgs& p, int64_t cus, int64_t bk) {
    if (std::min(p.m, p.n) <= 128) {
        const int64_t tiles = ((p.m + 127) / 128) * ((p.n + 127) / 128);
        const SplitPlan short_plan = splitk16_slices(p, 2 * cus, kSplit16ShortK, bk);
        if (short_plan.slices > 1 && tiles * short_plan.slices >= cus) return short_plan;
    }
    return splitk16_slices(p, 2 * cus, kSplit16MinK, bk);
}

template <typename T, int BM, int BN, int WM, int WN>
void launch_splitk16(const GemmArgs& p, const SplitPlan& plan, hipStream_t stream, int device) {
    using S = typename Elem<T>::storage;
    const int64_t mn = p.m * p.n;
    const int64_t slices = plan.slices;
    Workspace ws(static_cast<size_t>(slices * mn) * sizeof(float), device);
    GemmArgs q = p;
    q.batch = slices;
    q.k = plan.ks;
    q.k_total = p.k;
    q.stride_a = p.trans_a ? q.k * p.lda : q.k;  // slice s starts at k = s q.k
    q.stride_b = p.trans_b ? q.k : q.k * p.ldb;
    q.alpha = 1.0f;
    q.beta = 0.0f;
    q.cin = nullptr;
    q.c = ws.get();
    q.ldc = p.n;
    q.stride_c = mn;
    launch_config<T, BM, BN, WM, WN, true>(q, stream);
    const int64_t blocks = std::min<int64_t>((mn + kFinishBlock - 1) / kFinishBlock, 4 * int64_t{cu_count(device)});
    splitk_finish16_kernel<T><<<static_cast<unsigned>(blocks), kFinishBlock, 0, stream>>>(
        static_cast<const float*>(ws.get()), static_cast<int>(slices), p.m, p.n, p.alpha, p.beta,
        static_cast<const S*>(p.cin), p.cin_rs, p.cin_cs, static_cast<S*>(p.c), p.ldc);
    TP_AMD_HIP_CHECK(hipGetLastError());
}

// 16-bit types take the big tile when it still gives every CU a block;
// float32 (bound by its much slower MFMA rate) keeps the small one, whose
// registers fit without spilling.
template <typename T>
void launch_mfma(const GemmArgs& p, hipStream_t stream) {
    int device = 0;
    TP_AMD_HIP_CHECK(hipGetDevice(&device));
    if constexpr (std::is_same<T, float>::value) {
        const int cus = cu_count(device);
        const int batch_split = splitk32_small_batch(p, cus);
        if (batch_split > 1) {
            launch_splitk<64, 64, 2, 1>(p, batch_split, stream, device);
            return;
        }
        const int64_t tiles = ((p.m + 127) / 128) * ((p.n + 127) / 128) * p.batch;
        const int slices = splitk_slices(p, cus);
        // A [M, K] K-contiguous with B [K, N] N-contiguous (plain mm, and
        // the dX = dY W of a linear layer) is the slowest float32 layout;
        // the same product as C^T = B^T A^T reads B^T with its M axis
        // contiguous and A^T K-contiguous, the fastest one, and writes C
        // transposed.  Measured at 4096^3, after warm-up, on one box: 1077 us
        // this way, TT itself 1070 us; the NN kernel took 1257-1300 us.
        if (!p.trans_a && !p.trans_b && !p.trans_c && slices == 1 && !(p.batch == 1 && tiles * 4 <= cus)) {
            GemmArgs q = p;
            q.m = p.n;
            q.n = p.m;
            q.a = p.b;
            q.lda = p.ldb;
            q.stride_a = p.stride_b;
            q.trans_a = true;
            q.b = p.a;
            q.ldb = p.lda;
            q.stride_b = p.stride_a;
            q.trans_b = true;
            q.cin_rs = p.cin_cs;
            q.cin_cs = p.cin_rs;
            q.trans_c = true;
            launch_config<float, 128, 128, 2, 2>(q, stream);
            return;
        }
        if (p.batch == 1 && tiles * slices * 4 <= cus) {
            // A product that 128 x 128 tiles, even split over K, leave on
            // under a quarter of the CUs (config 1's 256^3: 4 tiles, 8
            // blocks): 64 x 64 tiles of two waves, split down to slices of
            // 64 of K.
            const int small = splitk_slices(p, cus, 64, 64);
            if (small > 1) {
                launch_splitk<64, 64, 2, 1>(p, small, stream, device);
            } else {
                launch_config<float, 64, 64, 2, 1>(p, stream);
            }
            return;
        }
        if (slices > 1) {
            launch_splitk<128, 128, 2, 2>(p, slices, stream, device);
            return;
        }
    }
    if constexpr (sizeof(typename Elem<T>::storage) == 2) {
        if (smallk::eligible<T>(p, cu_count(device))) {
            smallk::launch<T>(p, stream);
            return;
        }
        if (big::eligible<T>(p, cu_count(device))) {
            big::launch<T>(p, stream);
            return;
        }
        const int64_t big_tiles = ((p.m + 255) / 256) * ((p.n + 255) / 256) * p.batch;
        if (big_tiles >= cu_count(device)) {
            launch_config<T, 256, 256, 2, 4>(p, stream);
            return;
        }
        // Few 128 x 128 tiles and a long K (a Linear of a few hundred rows):
        // split K (splitk16_plan), up to two blocks a CU.  Measured
        // (bf16, this split against the tiles alone): 128 x 11008 x 4096
        // 36.4 against 57.7 us, 128 x 4096 x 4096 22.4 against 42.6 us,
        // 1024 x 1024 x 8192 41.5 against 81.4 us; 1024^3 in slices of 512
        // was slower (19.5 against 13.5 us) and is not split.
        const SplitPlan plan = splitk16_plan(p, cu_count(device), Mfma<T>::BK);
        if (plan.slices > 1) {
            launch_splitk16<T, 128, 128, 2, 2>(p, plan, stream, device);
            return;
        }
        // Too few 128 x 128 tiles for a quarter of the CUs (mm 1024^2 has
        // 64): 64 x 64 tiles of two waves.
        const int64_t tiles = ((p.m + 127) / 128) * ((p.n + 127) / 128) * p.batch;
        if (tiles * 4 <= cu_count(device)) {
            launch_config<T, 64, 64, 2, 1>(p, stream);
            return;
        }
    }
    launch_config<T, 128, 128, 2, 2>(p, stream);
}

// Products with an operand the matrix-core kernels cannot read in place (an
// odd K or leading dimension: a vocabulary of 50257, a Linear(1023, ...), a
// column slice at an odd offset) copy that operand into a dense K-major
// workspace [batch][M or N][K'], K' = K rounded up to the packet, with the
// columns K..K' zeroed.  An odd K alone only forces the K-major operands
// into such copies (their 16-byte packets run along K and would cross the
// end of a row); an operand stored with M or N contiguous stays where it
// is, since the bounds-checked tile loaders give zeros for its rows k >= K,
// and the product keeps K.  Before, an odd K repacked both operands: the
// dX = dY W of an LM head with a 50257 vocabulary (bf16 1 x 50257 x 4096)
// transposed the whole 400 MB weight on every call.  The copies cost a pass
// over the operands; the general kernel
// they replace runs ~16x slower than the matrix cores (2047^3 in bfloat16:
// 692 us there, 63 us repacked).  Products under kRepackMinMacs
// multiply-adds (about 160^3) keep the general kernel, which needs no
// workspace and no extra launches: measured, 130^3 is 2 us faster there and
// 200^3 7 us faster repacked.
constexpr double kRepackMinMacs = double(int64_t(1) << 22);

void check_status(int status) { TP_AMD_CHECK(status == 0, last_error()); }

template <typename T>
struct DtypeOf;
template <>
struct DtypeOf<float> { static constexpr int value = TP_AMD_FLOAT32; };
template <>
struct DtypeOf<bf16_t> { static constexpr int value = TP_AMD_BFLOAT16; };
template <>
struct DtypeOf<f16_t> { static constexpr int value = TP_AMD_FLOAT16; };

// A K-major source in one pass: dst row q (of bs x rows) = the source row
// (b, r) = (q / rows, q % rows) at src + b stride + r ld, elements 0..k, then
// zeros to kp.  A thread writes one 16-byte packet (kp is a whole number of
// them) from element loads, which are unaligned when ld or k is odd.
constexpr int kRepackBlock = 256;

template <typename S>
__global__ __launch_bounds__(kRepackBlock) void repack_rows_kernel(S* __restrict__ dst, const S* __restrict__ src,
                                                                   int64_t total, int64_t rows, int64_t ld,
                                                                   int64_t stride, int64_t k, int64_t kp) {
    constexpr int N = 16 / sizeof(S);
    const int64_t j0 = (static_cast<int64_t>(blockIdx.x) * kRepackBlock + threadIdx.x) * N;
    if (j0 >= kp) return;
    for (int64_t q = blockIdx.y; q < total; q += gridDim.y) {
        const S* row = src + (q / rows) * stride + (q % rows) * ld;
        S v[N];
#pragma unroll
        for (int e = 0; e < N; ++e) v[e] = j0 + e < k ? row[j0 + e] : S{};
        uint4 w;
        __builtin_memcpy(&w, v, 16);
        *reinterpret_cast<uint4*>(dst + q * kp + j0) = w;
    }
}

// x logical [bs][rows][k] (element (b, r, j) at x + b stride + r ld + j when
// K-major, + j ld + r otherwise) -> ws [bs][rows][kp], columns k..kp zero.
// K-major sources take repack_rows_kernel; the others the transpose copy and
// a fill of the padding.
template <typename S>
void repack_kmajor(int device, const void* x, int64_t ld, int64_t stride, bool kmajor, int64_t bs,
                   int64_t rows, int64_t k, int64_t kp, void* ws, hipStream_t stream) {
    constexpr int esize = sizeof(S);
    if (kmajor) {
        constexpr int N = 16 / esize;
        const int64_t total = bs * rows;
        const dim3 grid(static_cast<unsigned>((kp / N + kRepackBlock - 1) / kRepackBlock),
                        static_cast<unsigned>(std::min<int64_t>(total, 65535)));
        repack_rows_kernel<S><<<grid, kRepackBlock, 0, stream>>>(static_cast<S*>(ws), static_cast<const S*>(x),
                                                                 total, rows, ld, stride, k, kp);
        TP_AMD_HIP_CHECK(hipGetLastError());
        return;
    }
    const int64_t sizes[3] = {bs, rows, k};
    const int64_t dst[3] = {rows * kp, kp, 1};
    const int64_t src[3] = {stride, kmajor ? ld : 1, kmajor ? 1 : ld};
    check_status(tp_amd_launch_strided_copy(device, esize, 3, sizes, ws, dst, x, src));
    if (kp > k) {
        const uint64_t zero = 0;
        const int64_t pad[3] = {bs, rows, kp - k};
        check_status(tp_amd_launch_fill(device, esize, &zero, 3, pad, static_cast<char*>(ws) + k * esize, dst));
    }
}

template <typename T>
void launch_repacked(const GemmArgs& p, hipStream_t stream) {
    constexpr int V = Mfma<T>::V;
    constexpr int E = sizeof(typename Elem<T>::storage);
    int device = 0;
    TP_AMD_HIP_CHECK(hipGetDevice(&device));
    const int64_t kp = (p.k + V - 1) / V * V;
    const bool a_kmajor = !p.trans_a, b_kmajor = p.trans_b;
    // An in-place MN-major operand only needs its own packets aligned; for
    // the check K is taken as padded (its K extent is not read in packets).
    const bool fix_a = (a_kmajor && kp != p.k) || !operand_ok<T>(p.a, p.lda, p.stride_a, a_kmajor, p.m, kp);
    const bool fix_b = (b_kmajor && kp != p.k) || !operand_ok<T>(p.b, p.ldb, p.stride_b, b_kmajor, p.n, kp);
    // A batch-broadcast operand (stride 0) is copied once and stays broadcast.
    const int64_t bs_a = p.stride_a == 0 ? 1 : p.batch, bs_b = p.stride_b == 0 ? 1 : p.batch;
    const size_t bytes_a = fix_a ? static_cast<size_t>(bs_a * p.m * kp) * E : 0;
    const size_t off_b = (bytes_a + 255) / 256 * 256;
    const size_t bytes_b = fix_b ? static_cast<size_t>(bs_b * p.n * kp) * E : 0;
    Workspace ws(off_b + bytes_b, device);
    GemmArgs q = p;
    // Both operands copied: K' with zero terms on both sides (the big
    // kernels' whole K tiles apply).  Otherwise the in-place operand bounds
    // the product at K, and the copies' zero columns are never summed in.
    q.k = fix_a && fix_b ? kp : p.k;
    if (fix_a) {
        repack_kmajor<typename Elem<T>::storage>(device, p.a, p.lda, p.stride_a, !p.trans_a, bs_a, p.m, p.k, kp,
                                                 ws.get(), stream);
        q.a = ws.get();
        q.lda = kp;
        q.stride_a = p.stride_a == 0 ? 0 : p.m * kp;
        q.trans_a = false;
    }
    if (fix_b) {
        void* wb = static_cast<char*>(ws.get()) + off_b;
        repack_kmajor<typename Elem<T>::storage>(device, p.b, p.ldb, p.stride_b, p.trans_b, bs_b, p.n, p.k, kp, wb,
                                                 stream);
        q.b = wb;
        q.ldb = kp;
        q.stride_b = p.stride_b == 0 ? 0 : p.n * kp;
        q.trans_b = true;
    }
    // A thin product reads its repacked operand through the thin kernel.
    if (!launch_gemm_thin(DtypeOf<T>::value, q, stream)) launch_mfma<T>(q, stream);
}

template <typename T>
void launch_typed(const GemmArgs& p, hipStream_t stream) {
    if (mfma_eligible<T>(p)) {
        launch_mfma<T>(p, stream);
    } else if (p.k > 0 && tiles_fit(p) &&
               double(p.batch) * double(p.m) * double(p.n) * double(p.k) >= kRepackMinMacs) {
        launch_repacked<T>(p, stream);
    } else {
        launch_gemm_general<T>(p, stream);
    }
}

}  // namespace

bool splitk32_takes(const GemmArgs& p, int device) { return splitk32_small_batch(p, cu_count(device)) > 1; }

int64_t splitk16_blocks(const GemmArgs& p, int device, int64_t* slices) {
    const SplitPlan plan = splitk16_plan(p, cu_count(device), Mfma<bf16_t>::BK);
    const int64_t tiles = ((p.m + 127) / 128) * ((p.n + 127) / 128);
    *slices = plan.slices;
    return plan.slices > 1 ? tiles * plan.slices : 0;
}

void launch_gemm(int dtype, const GemmArgs& p, hipStream_t stream) {
    if (launch_gemm_thin(dtype, p, stream)) return;
    switch (dtype) {
        case TP_AMD_FLOAT32: launch_typed<float>(p, stream); break;
        case TP_AMD_BFLOAT16: launch_typed<bf16_t>(p, stream); break;
        case TP_AMD_FLOAT16: launch_typed<f16_t>(p, stream); break;
        default:
            TP_AMD_CHECK(false, "GEMM takes float32, float16 or bfloat16, got ", dtype_name(dtype));
    }
}

}  // namespace tp_amd
