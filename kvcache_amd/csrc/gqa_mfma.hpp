// gqa_mfma.hpp -- grouped-query decode on the matrix cores (fp16 K/V, head_dim 64/128).
//
// Included by decode_kernels.hpp inside namespace kvc::{anonymous}; uses its helpers.
//
// When one KV head serves a group of g > 2 query heads, the per-head VALU dot
// products of split_kernel cost ~g times more instructions per K/V byte and the
// kernel stops being bandwidth-bound.  Here one wave computes all heads of the
// group at once with v_mfma_f32_16x16x32_f16 (heads padded to 16):
//
//   QK^T : S[16 tok][16 heads] = K[16 tok][32 dims] x Q^T[32 dims][16 heads],
//          D/32 MFMAs per 16-token subtile.  The A operand (lane l: row l%16, 16
//          bytes at dim 8*(l/16) + 32j) would read half of 16 cache lines per load
//          instruction, which streams at about half the rate of whole lines when a
//          launch occupies few CUs; so K is loaded like V, 1 KiB of whole rows per
//          wave load, staged in LDS (16-byte chunks XOR-permuted by row & 7) and
//          read back in the operand layout.  The B operand is q in that layout
//          (loaded once per unit).
//   softmax: the result layout gives lane l the scores of head l%16 for tokens
//          4*(l/16)+r (r = 0..3) of each subtile, i.e. 8 scores per lane for a
//          32-token tile; the tile max per head needs two lane exchanges (xor 16,
//          xor 32, in registers with the permlane swaps); online (max, sum) per head
//          in log2 units.  Each tile's P V goes into a fresh accumulator, folded into
//          O with the rows' rescale factors afterwards, so the MFMAs do not wait for
//          the factors' lane gather.
//   PV   : O[16 heads][16 dims] += P[16 heads][32 tok] x V[32 tok][16 dims] per
//          16-dim column tile.  The A operand is the lane's own 8 probabilities
//          (token order tau(g, i) = 4g+i for i < 4, 16+4g+i-4 otherwise); the B
//          operand needs V transposed (8 tokens of one dim per lane), so each
//          wave stages its 32-token V tile in LDS, row-major with 32-byte segments
//          XOR-permuted by row, and reads it back with the transposing LDS read
//          (two per 16-dim column tile).
//
// Unit decomposition, partial records, arrival counters and merge modes are those
// of split_kernel (one unit = sequence x KV head x chunk, all query heads of the
// group).  The chunk's block ids come with a planned entry (up to 56, read with
// it) or are staged in LDS, so chunks may span up to kMfmaMaxChunkBlocks blocks;
// BLOCK must be a power of two >= 16 (each 16-token subtile lies inside one block,
// located by a shift and a mask, and is read through one buffer descriptor whose
// size admits only the valid rows).  The fused cross-chunk merge runs on every
// thread of the last-arriving workgroup (weights per chunk in LDS, then each
// thread accumulates one (head, dim) over up to 32 chunks per round of loads).

constexpr int kMfmaTile = 32;             // tokens per wave tile (two 16-row subtiles)
constexpr int kMfmaMaxChunkBlocks = 1024; // block ids staged per unit
constexpr int kMfmaMaxHeads = 16;         // query heads per KV head on this path
constexpr int kMaxFusedChunks = 64;       // chunks the fused merge combines (one per lane)

typedef _Float16 f16x8v __attribute__((ext_vector_type(8)));
typedef short s16x4v __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16 (gfx950) at an LDS address held in a generic pointer.
__device__ __forceinline__ s16x4v ds_read_tr16(const char* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4v*)(__attribute__((address_space(3))) char*)(const_cast<char*>(p)));
}

template <int D, int MODE, int WPB>
__global__ __launch_bounds__(WPB * kWave) void gqa_mfma_kernel(const int* __restrict__ work, int work_ints, DecodeParams p_arg) {
    const DecodeParams& p = p_arg;
    static_assert(D == 64 || D == 128, "MFMA decode is built for head_dim 64 and 128");
    constexpr int ROW = D * 2;                 // bytes per fp16 K/V row
    constexpr int KJ = D / 32;                 // MFMA k-steps over the head dimension
    constexpr int NT = D / 16;                 // 16-dim output column tiles
    constexpr int VL = 16 * ROW / 1024;        // 1 KiB wave loads per 16-row V subtile
    constexpr bool SELF = MODE == kSelfPlanned || MODE == kSelfContig;
    constexpr bool PLANNED = MODE == kPlannedUniform || SELF;
    constexpr bool CONTIG = MODE == kContiguous || MODE == kSelfContig;
    constexpr bool PAGED = !CONTIG;
    // prompt attention: the 16 columns are 16 consecutive queries of one head (not
    // the heads of one query); query q attends to positions 0 .. fixed_len + q
    constexpr bool CAUSAL = MODE == kCausalTile;
    constexpr int kTileBytes = kMfmaTile * ROW;
    constexpr int kMainBytes = 2 * WPB * kTileBytes;   // per wave: V tile, then K tile
    __shared__ __attribute__((aligned(16))) char s_buf[kMainBytes];
    __shared__ int s_tab[PAGED ? kMfmaMaxChunkBlocks : 1];
    __shared__ float s_w[kMfmaMaxHeads][kMaxFusedChunks];
    __shared__ float s_L[kMfmaMaxHeads];
    __shared__ int s_last;
    __shared__ std::conditional_t<SELF, SelfPlanLds<kSelfMaxNMfma, WPB>, char> s_plan;

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = uniform(tid >> 6);
    const int heads = p.group;   // query heads of the KV group, <= 16 (host-checked)

    // One unit, given its entry header (hdr) and, on the host-planned path, the
    // entry's block ids (ev: one int per lane after the 8-int header).
    auto run_unit = [&](const int (&hdr)[8], const int ev) {
    // self-planned (persistent) launches: the parameters and per-lane indices are
    // derived anew in every unit, not hoisted out of the loop and held across it
    const DecodeParams p = SELF ? fresh_params() : p_arg;
    int tid_u = tid;
    if constexpr (SELF) asm volatile("" : "+v"(tid_u));
    const int lane = tid_u & (kWave - 1);
    const int n16 = lane & 15;   // head (S layout) / output column within a tile
    const int g4 = lane >> 4;    // lane group
    Unit u;
    int qh = 0, q0 = 0;  // causal: query head and first query of the tile
    if constexpr (CAUSAL) {
        int unit = blockIdx.x;
        const int ntq = (p.N + 15) / 16;
        qh = unit % p.Hq;  unit /= p.Hq;
        q0 = (ntq - 1 - unit % ntq) * 16;  unit /= ntq;  // longest prefixes first
        u.c = unit;
        u.s = 0;
        u.sub = 0;
        u.hk = qh / p.group;
        u.tab_start = PAGED && p.tab_off ? p.tab_off[0] : 0;
        const int lmax = min(p.fixed_len + min(q0 + 16, p.N), p.cap);  // keys of the tile's last query
        u.j0 = u.c * p.chunk_tokens;
        u.j1 = min(u.j0 + p.chunk_tokens, lmax);
        if (u.c >= p.max_chunks || u.j0 >= lmax) return;
        u.nc = (lmax + p.chunk_tokens - 1) / p.chunk_tokens;  // chunks of the tile's last query
        u.rec0 = 0; u.cstride = 0; u.ctr_idx = 0;
    } else {
        if (!load_unit<PLANNED, PAGED>(p, hdr, heads, u)) {
            if (u.over_cap) nan_rows<_Float16, D, WPB * kWave>(p, u.s, u.hk * p.group, heads);
            return;
        }
    }
    const int s = u.s, hk = u.hk, j0 = u.j0, j1 = u.j1, nc = u.nc;
    const int hq0 = hk * p.group;
    const int rows = CAUSAL ? 16 : heads;  // output rows of the unit's 16-column block
    const int ntiles = (j1 - j0 + kMfmaTile - 1) / kMfmaTile;
    const int kmax = wave < ntiles ? (ntiles - wave + WPB - 1) / WPB : 0;

    // Fused append (planned launches): the chunk holding the step's new row uses
    // the new K/V in place of the pool's (this lane's slices of it, loaded here,
    // ahead of the table), and the unit of the first head subgroup stores the row
    // in the pool once the block ids are staged.
    // The position is loaded here but resolved only after the first K/V tile is in
    // flight (resolve_append): nothing before the first loads waits for it.
    int wp = -1, w_raw = -1;
    u32x4 vnew = {0, 0, 0, 0}, kst = {0, 0, 0, 0};  // bytes (lane*16) % ROW of the new V and K rows
    if constexpr (PLANNED) {
        if (p.wpos != nullptr) {
            const char* kn = static_cast<const char*>(p.k_new) + ((size_t)s * p.Hkv + hk) * ROW;
            const char* vn = static_cast<const char*>(p.v_new) + ((size_t)s * p.Hkv + hk) * ROW;
            vnew = *reinterpret_cast<const u32x4*>(vn + (lane * 16) % ROW);
            kst = *reinterpret_cast<const u32x4*>(kn + (lane * 16) % ROW);
            w_raw = p.wpos[s];
        }
    }

    // q as the B operand of QK^T: lane l holds head l%16, dims 8*(l/16) + 32j .. +7;
    // heads past the group read as zero through the descriptor bound.
    f16x8v qb[KJ];
    if constexpr (CAUSAL) {
        // lane l holds query q0 + l%16 of head qh; queries past N read as zero
        const __amdgpu_buffer_rsrc_t qr = tile_rsrc(p.q, p.N * p.Hq * ROW);
        const int qoff = ((q0 + n16) * p.Hq + qh) * ROW + g4 * 16;
#pragma unroll
        for (int j = 0; j < KJ; ++j) qb[j] = __builtin_bit_cast(f16x8v, buffer_load16(qr, qoff + j * 64));
    } else {
        const char* qbase = static_cast<const char*>(p.q) + ((size_t)s * p.Hq + hq0) * ROW;
        const __amdgpu_buffer_rsrc_t qr = tile_rsrc(qbase, heads * ROW);
#pragma unroll
        for (int j = 0; j < KJ; ++j)
            qb[j] = __builtin_bit_cast(f16x8v, buffer_load16(qr, n16 * ROW + g4 * 16 + j * 64));
    }
    const int qlast = CAUSAL ? p.fixed_len + q0 + n16 : INT_MAX;  // last key this column may see
    // scores use |scale|: a negative scale negates q instead (exact in fp16)
    const float sl2 = fabsf(p.scale_log2);
    if (p.scale_log2 < 0.f) {
#pragma unroll
        for (int j = 0; j < KJ; ++j) qb[j] = -qb[j];
    }

    const char* kb = static_cast<const char*>(p.k);
    const char* vb = static_cast<const char*>(p.v);
    size_t cbase = 0;
    // paged: BLOCK is a power of two (host-checked), so block index and offset are
    // a shift and a mask
    const int bsh = PAGED ? __builtin_ctz((unsigned)p.block) : 0, bmask = p.block - 1;
    const int b0 = PAGED ? j0 >> bsh : 0;
    int nblk = 0;
    bool inl = false;  // block ids from the entry (no table read, no LDS staging)
    if constexpr (CONTIG) {
        cbase = ((size_t)s * p.seq_stride + (size_t)hk * p.head_stride) * 2;
    } else {
        nblk = min(j1 > j0 ? ((j1 - 1) >> bsh) - b0 + 1 : 0, kMfmaMaxChunkBlocks);
        inl = PLANNED && p.work_ints == kWave && u.n_inline >= nblk;
        if (!inl) {
            const int first = u.tab_start + (PLANNED ? 0 : b0);
            const __amdgpu_buffer_rsrc_t trs =
                PLANNED ? tile_rsrc(p.table_all, p.table_len * 4) : tile_rsrc(p.table_all + first, nblk * 4);
            const int tb = PLANNED ? first * 4 : 0;
            for (int b = tid; b < nblk; b += WPB * kWave)
                s_tab[b] = (int)__builtin_amdgcn_raw_buffer_load_b32(trs, tb + b * 4, 0, 0);
            __syncthreads();
        }
    }
    // physical block of the chunk's rel-th block (rel uniform, < nblk), as a scalar
    // from either source
    auto block_id = [&](int rel) -> int {
        if (inl) return __builtin_amdgcn_readlane(ev, 8 + min(rel, kWave - 9));
        return uniform(s_tab[min(rel, kMfmaMaxChunkBlocks - 1)]);
    };
    // The step's new row: its position within this chunk (else -1), and its store into
    // the pools by the first head subgroup.  No tile of this unit reads the pools'
    // copy of that row (consume takes it from the inputs), so the store may land
    // after the unit's loads.
    auto resolve_append = [&]() {
        if constexpr (PLANNED) {
            if (p.wpos != nullptr) wp = uniform((w_raw >= j0 && w_raw < j1) ? w_raw : -1);
        }
        if (PLANNED && wp >= 0 && u.sub == 0 && wave == 0 && lane < ROW / 16) {
            const int phys = block_id(max((wp >> bsh) - b0, 0));
            const size_t off = ((size_t)(phys * p.Hkv + hk) * p.block + (wp & bmask)) * ROW + lane * 16;
            *reinterpret_cast<u32x4*>(const_cast<char*>(kb) + off) = kst;
            *reinterpret_cast<u32x4*>(const_cast<char*>(vb) + off) = vnew;
        }
    };

    struct Tile {
        u32x4 k[2][VL];   // both: 1 KiB of whole rows per wave load
        u32x4 v[2][VL];
    };
    // Byte offset of the 16-row subtile starting at token t (inside one block).  All
    // of the tile addressing stays in scalar registers: a vector temporary here can
    // land on a register whose load is still in flight and make the issue wait.
    const unsigned blk_bytes = (unsigned)p.block * ROW;
    auto subtile = [&](int t) -> size_t {
        if constexpr (CONTIG) {
            return cbase + (size_t)t * ROW;
        } else {
            const int rel = min(max((t >> bsh) - b0, 0), max(nblk - 1, 0));
            const unsigned slot = (unsigned)(block_id(rel) * p.Hkv + hk);
            return (size_t)slot * blk_bytes + (unsigned)((t & bmask) * ROW);
        }
    };
    auto issue = [&](int k, Tile& T) {
        const int t0 = j0 + (wave + WPB * k) * kMfmaTile;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int t = t0 + 16 * h;
            // valid rows, never past the end of the block holding the subtile (the
            // empty asm keeps the clamp from turning into a vector med3)
            int rows = max(j1 - t, 0);
            asm("" : "+s"(rows));
            rows = min(rows, 16);
            if constexpr (PAGED) rows = min(rows, p.block - (t & bmask));
            const size_t off = rows > 0 ? subtile(t) : 0;
            const __amdgpu_buffer_rsrc_t kr = tile_rsrc(kb + off, rows * ROW);
            const __amdgpu_buffer_rsrc_t vr = tile_rsrc(vb + off, rows * ROW);
#pragma unroll
            for (int q = 0; q < VL; ++q) T.k[h][q] = buffer_load16(kr, q * 1024 + lane * 16);
#pragma unroll
            for (int q = 0; q < VL; ++q) T.v[h][q] = buffer_load16(vr, q * 1024 + lane * 16);
        }
    };

    char* vt = s_buf + wave * kTileBytes;           // this wave's V tile
    char* kt = s_buf + (WPB + wave) * kTileBytes;   // and K tile
    // 32-byte segment of a V row in LDS: the sixteen rows one transposing read
    // touches (4 g4 + r, same segment) spread over all banks
    auto vseg = [](int r, int seg) { return seg ^ (D == 64 ? (r >> 1) & 3 : r & 7); };
    // 16-byte chunk of a K row in LDS: the sixteen rows one operand read touches
    // (same chunk) spread over the banks
    auto kchunk = [](int r, int c) { return c ^ (r & 7); };
    float m = -FLT_MAX, l = 0.f;            // per head n16 (identical in the four lane groups)
    f32x4 O[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) O[nt] = f32x4{0.f, 0.f, 0.f, 0.f};

    // FULL: every row of the tile is a valid key for every column and none is the
    // step's new row, so the masks and the new-row selects drop out
    auto consume = [&](int k, const Tile& T, auto full_tag) {
        constexpr bool FULL = decltype(full_tag)::value;
        const int t0 = j0 + (wave + WPB * k) * kMfmaTile;
        // V rows -> LDS, row-major with the row's 32-byte segments (16 dims each)
        // permuted by vseg
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int q = 0; q < VL; ++q) {
                const int off = q * 1024 + lane * 16;
                const int r = 16 * h + off / ROW;
                const int cb = off % ROW;
                *reinterpret_cast<u32x4*>(vt + r * ROW + vseg(r, cb >> 5) * 32 + (cb & 31)) =
                    !FULL && t0 + r == wp ? vnew : T.v[h][q];
                *reinterpret_cast<u32x4*>(kt + r * ROW + kchunk(r, cb >> 4) * 16) = !FULL && t0 + r == wp ? kst : T.k[h][q];
            }
        __builtin_amdgcn_wave_barrier();
        asm volatile("" ::: "memory");
        // scores of the 32 tokens for all heads; A operand from the K tile: row
        // 16h + n16, dims 8*g4 + 32j .. +7 (16-byte chunk g4 + 4j)
        f32x4 S[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int r = 16 * h + n16;
            f16x8v ka[KJ];
#pragma unroll
            for (int j = 0; j < KJ; ++j) ka[j] = *reinterpret_cast<const f16x8v*>(kt + r * ROW + kchunk(r, g4 + 4 * j) * 16);
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < KJ; ++j) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[j], qb[j], acc, 0, 0, 0);
            S[h] = acc;
        }
        // the scale is >= 0 here (q carries its sign), so the tile max is taken on
        // the raw scores and each probability is one fma and one exp2
        bool ok[8];
        float mx = -FLT_MAX;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int h = i >> 2, r = i & 3;
            ok[i] = FULL || (t0 + 16 * h + 4 * g4 + r < j1 && t0 + 16 * h + 4 * g4 + r <= qlast);
            mx = ok[i] ? fmaxf(mx, S[h][r]) : mx;
        }
        mx = max_xor32(max_xor16(mx));
        const float mn = fmaxf(m, mx * sl2);
        const float corr = fast_exp2(m - mn);
        float ps = 0.f;
        f16x8v pa;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float pi = ok[i] ? fast_exp2(__builtin_fmaf(S[i >> 2][i & 3], sl2, -mn)) : 0.f;
            ps += pi;
            pa[i] = (_Float16)pi;
        }
        l = __builtin_fmaf(l, corr, ps);
        m = mn;
        // rescale factors of the output rows: row 4*g4 + r belongs to head 4*g4 + r,
        // whose factor is held by lane 4*g4 + r (applied after this tile's P V, which
        // is computed into its own accumulator and so does not wait for them)
        float cr[4];
#pragma unroll
        for (int r = 0; r < 4; ++r)
            cr[r] = __int_as_float(__builtin_amdgcn_ds_bpermute((4 * g4 + r) << 2, __float_as_int(corr)));
        __builtin_amdgcn_wave_barrier();
        asm volatile("" ::: "memory");
        // V^T operand: 8 tokens tau(g4, i) of dim n16 + 16 nt, by two transposing
        // reads.  ds_read_b64_tr_b16 over a group of 16 lanes: lane i receives element
        // i % 4 of the 8 bytes addressed by lane 4j + i/4, for j = 0..3.  Lane 4r + c
        // of group g4 addresses dims 16 nt + 4c .. +3 of token 4 g4 + r (then of token
        // 16 + 4 g4 + r), so lane n16 receives dim 16 nt + n16 of those four tokens.
        const int vr0 = 4 * g4 + (n16 >> 2);
        const int vcb = 8 * (n16 & 3);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const s16x4v lo = ds_read_tr16(vt + vr0 * ROW + vseg(vr0, nt) * 32 + vcb);
            const s16x4v hi = ds_read_tr16(vt + (vr0 + 16) * ROW + vseg(vr0 + 16, nt) * 32 + vcb);
            const f16x8v vbv = __builtin_bit_cast(f16x8v, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
            const f32x4 pv = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, vbv, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r) O[nt][r] = __builtin_fmaf(O[nt][r], cr[r], pv[r]);
        }
        __builtin_amdgcn_wave_barrier();
        asm volatile("" ::: "memory");
    };

    auto step = [&](int k, const Tile& T) {
        const int t0 = j0 + (wave + WPB * k) * kMfmaTile;
        const bool full = t0 + kMfmaTile <= j1 && (!CAUSAL || t0 + kMfmaTile - 1 <= p.fixed_len + q0) &&
                          (wp < t0 || wp >= t0 + kMfmaTile);
        if (full) consume(k, T, std::true_type{});
        else consume(k, T, std::false_type{});
    };
    if (kmax > 0) {
        Tile A, B;
        issue(0, A);
        resolve_append();
        for (int k = 0;; k += 2) {
            issue(k + 1, B);
            step(k, A);
            if (k + 1 >= kmax) break;
            issue(k + 2, A);
            step(k + 1, B);
            if (k + 2 >= kmax) break;
        }
    } else {
        resolve_append();
    }
    l = sum_xor32(sum_xor16(l));

    // Combine the waves: per-wave (m, l) per head and O through LDS.  Only the first
    // nwa waves held tiles (they are dealt round-robin); the others hold (m, l, O) =
    // (-FLT_MAX, 0, 0), whose weight exp2(-FLT_MAX - M) is 0, so leaving them out of
    // the sums changes no bit of the result.
    const int nwa = min(WPB, ntiles);
    // Each wave writes its partials over its own V tile (16 heads x D floats: exactly
    // one tile) and K tile ((m, l) per head), which only it used, so one barrier
    // (every wave's partials written) is enough.
    static_assert(kMfmaMaxHeads * D * 4 == kTileBytes && kMfmaMaxHeads * 2 * 4 <= kTileBytes, "partials fit the tiles");
    auto acc_of = [&](int w) { return reinterpret_cast<const float*>(s_buf + w * kTileBytes); };        // [16][D]
    auto ml_of = [&](int w) { return reinterpret_cast<const float*>(s_buf + (WPB + w) * kTileBytes); };  // [16][2]
    if (wave < nwa) {
        float* my_acc = reinterpret_cast<float*>(vt);
        float* my_ml = reinterpret_cast<float*>(kt);
        if (lane < 16) {
            my_ml[lane * 2] = m;
            my_ml[lane * 2 + 1] = l;
        }
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int r = 0; r < 4; ++r) my_acc[(4 * g4 + r) * D + n16 + 16 * nt] = O[nt][r];
    }
    __syncthreads();

    _Float16* ob = static_cast<_Float16*>(p.out) + ((size_t)s * p.Hq + hq0) * D;
    const bool atomic_parts = p.merge_mode == kMergeAtomic;
    if constexpr (CAUSAL) {
        // row g is query q0 + g: written directly when its keys fit one chunk, else as
        // chunk record ((q * max_chunks + c) * Hq + qh) for the merge kernel
        for (int idx = tid; idx < 16 * D; idx += WPB * kWave) {
            const int g = idx / D, d = idx % D, q = q0 + g;
            if (q >= p.N) continue;
            const int ncq = (min(p.fixed_len + q + 1, p.cap) + p.chunk_tokens - 1) / p.chunk_tokens;
            if (u.c >= ncq) continue;  // this chunk lies past the query's keys
            float M = -FLT_MAX;
#pragma unroll
            for (int w = 0; w < WPB; ++w)
                if (w < nwa) M = fmaxf(M, ml_of(w)[g * 2]);
            float lt = 0.f, at = 0.f;
#pragma unroll
            for (int w = 0; w < WPB; ++w) {
                if (w >= nwa) break;
                const float wt = fast_exp2(ml_of(w)[g * 2] - M);
                lt = __builtin_fmaf(wt, ml_of(w)[g * 2 + 1], lt);
                at = __builtin_fmaf(wt, acc_of(w)[g * D + d], at);
            }
            if (ncq == 1) {
                static_cast<_Float16*>(p.out)[((size_t)q * p.Hq + qh) * D + d] =
                    (_Float16)(lt > 0.f ? at * (1.0f / lt) : 0.f);
            } else {
                const size_t rec = ((size_t)q * p.max_chunks + u.c) * p.Hq + qh;
                p.part_acc[rec * D + d] = at;
                if (d == 0) {
                    p.part_ml[rec * 2] = M;
                    p.part_ml[rec * 2 + 1] = lt;
                }
            }
        }
        return;  // split queries are merged by merge_kernel
    }
    for (int idx = tid; idx < rows * D; idx += WPB * kWave) {
        const int g = idx / D, d = idx % D;
        float M = -FLT_MAX;
#pragma unroll
        for (int w = 0; w < WPB; ++w)
            if (w < nwa) M = fmaxf(M, ml_of(w)[g * 2]);
        float lt = 0.f, at = 0.f;
#pragma unroll
        for (int w = 0; w < WPB; ++w) {
            if (w >= nwa) break;
            const float wt = fast_exp2(ml_of(w)[g * 2] - M);
            lt = __builtin_fmaf(wt, ml_of(w)[g * 2 + 1], lt);
            at = __builtin_fmaf(wt, acc_of(w)[g * D + d], at);
        }
        if (nc == 1) {
            ob[(size_t)g * D + d] = (_Float16)(lt > 0.f ? at * (1.0f / lt) : 0.f);
        } else {
            const size_t rec = u.rec0 + g;
            if (atomic_parts) {
                __hip_atomic_store(p.part_acc + rec * D + d, at, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (d == 0) {
                    __hip_atomic_store(p.part_ml + rec * 2, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(p.part_ml + rec * 2 + 1, lt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            } else {
                p.part_acc[rec * D + d] = at;
                if (d == 0) {
                    p.part_ml[rec * 2] = M;
                    p.part_ml[rec * 2 + 1] = lt;
                }
            }
        }
    }
    if (nc == 1 || p.merge_mode == kMergeKernel) return;

    // Fused merge: every thread's partial stores complete, then one arrival per unit.
    if (atomic_parts) {
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
    } else {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    }
    __syncthreads();
    unsigned long long* ctr = p.counters + ctr_slot(u.ctr_idx, p.ctr_shift);
    if (tid == 0) s_last = arrive(ctr, p.epoch) == (unsigned)(nc - 1);
    __syncthreads();
    if (!s_last) return;
    if (!atomic_parts) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    auto ld = [&](const float* a) {
        return atomic_parts ? __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : *a;
    };
    const size_t first = u.rec0 - (size_t)u.c * u.cstride;  // record of chunk 0, head 0
    const int ncm = min(nc, kMaxFusedChunks);                // the host keeps nc within this
    // per head: chunk weights 2^(m_c - M) (one chunk per lane) and the total sum; m and
    // l are read together, unconditionally (lanes past the count re-read the last chunk
    // and drop out by select)
    for (int g = wave; g < heads; g += WPB) {
        const bool in = lane < ncm;
        const size_t rec = first + (size_t)min(lane, ncm - 1) * u.cstride + g;
        const float mraw = ld(p.part_ml + rec * 2), lraw = ld(p.part_ml + rec * 2 + 1);
        const float mc = in ? mraw : -FLT_MAX;
        float M = mc;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) M = fmaxf(M, shfl_xor(M, o));
        const float w = in ? fast_exp2(mc - M) : 0.f;
        float lw = in ? w * lraw : 0.f;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) lw += shfl_xor(lw, o);
        s_w[g][lane] = w;
        if (lane == 0) s_L[g] = lw;
    }
    __syncthreads();
    // each thread owns one (head, dim) and reads its chunk partials E at a time (one
    // round for up to 32 chunks): loads unconditional (indices clamped to the last
    // chunk, weights of chunks past the count are 0), E fixed per variant so that no
    // branch sits between the loads
    auto merge_out = [&](auto e_tag) {
        constexpr int E = decltype(e_tag)::value;
        for (int idx = tid; idx < heads * D; idx += WPB * kWave) {
            const int g = idx / D, d = idx % D;
            float acc[4] = {0.f, 0.f, 0.f, 0.f};
            for (int c0 = 0; c0 < ncm; c0 += E) {
                float a[E];
#pragma unroll
                for (int e = 0; e < E; ++e)
                    a[e] = ld(p.part_acc + (first + (size_t)min(c0 + e, ncm - 1) * u.cstride + g) * D + d);
#pragma unroll
                for (int e = 0; e < E; ++e)
                    acc[e & 3] = __builtin_fmaf(c0 + e < ncm ? s_w[g][c0 + e] : 0.f, a[e], acc[e & 3]);
            }
            const float sum = (acc[0] + acc[1]) + (acc[2] + acc[3]);
            const float L = s_L[g];
            ob[(size_t)g * D + d] = (_Float16)(L > 0.f ? sum * (1.0f / L) : 0.f);
        }
    };
    // (head_dim 128 keeps 16-chunk rounds: its main loop already fills the registers)
    if (D == 128 || ncm <= 16) merge_out(std::integral_constant<int, 16>{});
    else merge_out(std::integral_constant<int, 32>{});
    if (tid == 0) __hip_atomic_store(ctr, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };  // run_unit

    if constexpr (SELF) {
        // self-planned launches pass the device lengths as the (preloaded) first argument
        self_plan_loop<_Float16, D, WPB * kWave>(work, work_ints, s_plan, heads,
                                                 [&](const int (&hdr)[8]) { run_unit(hdr, 0); },
                                                 [] { return false; }, [] {});
    } else {
        // planned entries carry the unit's block ids after the 8-int header (one int
        // per lane): entry and header are read first, from the preloaded arguments
        int ev = 0;
        int hdr[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if constexpr (PLANNED) {
            if (work_ints == kWave) ev = work[(size_t)blockIdx.x * kWave + lane];
            read_header(work, work_ints, hdr);
        } else if constexpr (!CAUSAL) {
            read_seq<PAGED>(p, hdr);
        }
        run_unit(hdr, ev);
    }
}
