// gemm.hip -- host side of the fused fp32 MFMA GEMM for gfx950 (pxk_gemm, include/pxk.h): the
// tile and split-K planner, argument checks and launches, and the allocation-free variant. The
// kernels are in gemm_impl.hpp, instantiated by gemm_tab_*.hip.
#include "gemm_impl.hpp"

namespace pxk {
namespace {

const Table kTables[] = {{kTable0, kTable0Size}, {kTable1, kTable1Size}, {kTable2, kTable2Size},
                         {kTable3, kTable3Size}, {kTable4, kTable4Size}, {kTable5, kTable5Size}};

// Plan index <-> PXK_TILE_*: the MFMA tiles in table order, the skinny kernels after them.
constexpr int kSkinnyTile = kTiles;
int public_tile(int t) {
    if (t < 6) return t + 1;
    if (t == 6) return PXK_TILE_32x48_DIRECT;
    return t == 7 ? PXK_TILE_32x48 : PXK_TILE_SKINNY;
}
int plan_tile(int id) {  // -1: none
    if (id >= PXK_TILE_128x128 && id <= PXK_TILE_32x32_DIRECT) return id - 1;
    if (id == PXK_TILE_32x48_DIRECT) return 6;
    if (id == PXK_TILE_32x48) return 7;
    return id == PXK_TILE_SKINNY ? kSkinnyTile : -1;
}

struct TileInfo {
    int bm, bn, bk, threads, smem_bytes;
    double floor_us;  // a K stage of a workgroup alone on its CU (load latency bound), measured
    double util;      // MFMA utilisation when several waves share a SIMD, measured
    bool direct;      // waves stream their operands from L2 into registers (no LDS panels)
};

template <class C>
constexpr int smem_of() {
    // The largest of the four (TA, TB) layouts: what a CU must hold for one workgroup.
    int s = Layout<C, false, false>::SIZE;
    if (Layout<C, false, true>::SIZE > s) s = Layout<C, false, true>::SIZE;
    if (Layout<C, true, false>::SIZE > s) s = Layout<C, true, false>::SIZE;
    if (Layout<C, true, true>::SIZE > s) s = Layout<C, true, true>::SIZE;
    return 4 * s;
}

const TileInfo kTileInfo[kTiles] = {
    {128, 128, 32, C128::NT, smem_of<C128>(), 1.0, 0.75, false},
    {64, 64, 32, C64::NT, smem_of<C64>(), 0.8, 0.65, false},
    {32, 64, 64, C32x64::NT, smem_of<C32x64>(), 0.8, 0.55, false},
    {32, 32, 64, C32::NT, smem_of<C32>(), 0.8, 0.5, false},
    {32, 64, 64, C32x64::NT, 4 * C32x64::KS * 32 * C32x64::LDC, 0.65, 0.55, true},
    {32, 32, 64, C32::NT, 4 * C32::KS * 32 * C32::LDC, 0.65, 0.5, true},
    {32, 48, 64, C32x48::NT, 4 * C32x48::KS * 32 * C32x48::LDC, 0.65, 0.55, true},
    {32, 48, 64, C32x48::NT, smem_of<C32x48>(), 0.8, 0.55, false},
};

constexpr int kSkinnyMaxLds = 64 * 1024;

int skinny_mb(int64_t m) { return m <= 4 ? 4 : (m <= 8 ? 8 : 16); }

// The NT kernel's LDS: A (MB x K rounded up to 64) and the MB x 68 output tile.
size_t skinny_nt_lds(const pxk_gemm_desc* d) {
    const int64_t mb = skinny_mb(d->m), kp = cdiv(d->k, 64) * 64;
    return static_cast<size_t>(mb * kp + mb * kSkinnyLDC) * sizeof(float);
}

// Whether the descriptor is one the skinny kernels compute: up to 16 rows of an unbatched,
// untransposed A, no prologue or causal range, one of the built (layout, epilogue) pairs.
const SkinnyEntry* skinny_entry(const pxk_gemm_desc* d) {
    if (d->m > 16 || d->k <= 0 || d->batch != 1 || d->kgroups != 1 || d->causal != PXK_CAUSAL_NONE ||
        d->prologue != PXK_PRO_NONE || d->trans_a != 0)
        return nullptr;
    for (int i = 0; i < kSkinnySize; ++i) {
        const SkinnyEntry& e = kSkinny[i];
        if (e.tb == (d->trans_b != 0) && e.epi == d->epilogue) {
            if (e.tb && (d->splits > 1 || skinny_nt_lds(d) > kSkinnyMaxLds)) return nullptr;
            return &e;
        }
    }
    return nullptr;
}

const Entry* find_entry(int ta, int tb, int pro, int epi) {
    for (const Table& t : kTables)
        for (int i = 0; i < t.n; ++i) {
            const Entry& e = t.e[i];
            if (e.ta == ta && e.tb == tb && e.pro == pro && e.epi == epi) return &e;
        }
    return nullptr;
}

Op to_op(const pxk_operand& o) {
    return Op{o.ptr, o.ld, o.batch_stride, o.inner_stride, o.inner_div, o.group_stride};
}

bool vec_ok(const pxk_operand& o, int64_t contiguous_extent) {
    if (o.ptr == nullptr) return true;
    return aligned16(o.ptr) && o.ld % 4 == 0 && o.batch_stride % 4 == 0 && o.inner_stride % 4 == 0 &&
           o.group_stride % 4 == 0 && contiguous_extent % 4 == 0;
}

struct Plan {
    const Entry* e;
    const SkinnyEntry* skinny;  // set when tile == kSkinnyTile
    int tile, splits;
    int64_t tiles_m, tiles_n;
    int64_t kc;  // skinny NN: K rows per split; skinny NT: K rounded up to 64
    int width;   // skinny: columns per workgroup
};

bool rope_fits(const pxk_gemm_desc* d, int bn) {
    return d->n <= bn || bn % d->head_dim == 0;
}

// Output tiles a launch computes (TRI skips those strictly above the diagonal).
int64_t live_tiles(const pxk_gemm_desc* d, int bm, int bn) {
    const int64_t tm = cdiv(d->m, bm), tn = cdiv(d->n, bn);
    if (d->causal != PXK_CAUSAL_TRI) return tm * tn * d->batch;
    int64_t t = 0;
    for (int64_t i = 0; i < tm; ++i) {
        const int64_t lim = (i * bm + bm - 1) / bn + 1;
        t += lim < tn ? lim : tn;
    }
    return t * d->batch;
}

// K stages of the longest tile (K_LE_M / K_GE_M tiles see a triangular share of K; the slowest
// one bounds the launch).
double max_stages(const pxk_gemm_desc* d, int bm, int bk) {
    const int64_t tm = cdiv(d->m, bm);
    if (d->causal == PXK_CAUSAL_NONE || d->causal == PXK_CAUSAL_TRI)
        return static_cast<double>(cdiv(d->k, bk)) * static_cast<double>(d->kgroups);
    int64_t most = 0;
    for (int64_t i = 0; i < tm; ++i) {
        int64_t lo = 0, hi = d->k;
        if (d->causal == PXK_CAUSAL_K_LE_M) hi = i * bm + bm < d->k ? i * bm + bm : d->k;
        if (d->causal == PXK_CAUSAL_K_GE_M) lo = i * bm < d->k ? i * bm : d->k;
        const int64_t st = hi > lo ? cdiv(hi - lo, bk) : 0;
        if (st > most) most = st;
    }
    return static_cast<double>(most) * static_cast<double>(d->kgroups);
}

// Estimated microseconds of one launch on 256 CUs (4 SIMDs each, ~2.4 GHz), calibrated on the
// 512-token GEMMs of a 576-wide model and its 49152-entry LM head: a fixed launch/prologue/epilogue
// cost, then per K stage the larger of the tile's latency floor and the MFMA time of the waves that
// share a SIMD; split-K adds the reduction launch and the partials' round trip through HBM.
double estimate(const pxk_gemm_desc* d, const TileInfo& t, double tiles, double stages, int splits) {
    const double per = std::ceil(stages / splits);
    const double waves_per_simd = std::ceil(tiles * splits / 256.0);
    const double mfma_us = static_cast<double>(t.bm) * t.bn * t.bk / 128.0 / 2400.0;
    double floor = t.floor_us, util = t.util;
    if (t.direct && d->trans_b && d->prologue != PXK_PRO_NONE) {
        // An NT relevance GEMM with the stabilised-divide prologue streams A, Z and B as K-contiguous
        // rows, each 16-lane group reading 16 rows x 64 B per instruction: at 512 rows the direct
        // tiles run 10-25% slower than from LDS panels (measured; without the prologue they win).
        floor = 1.0;
        util *= 0.65;
    } else if (t.direct && d->trans_b && waves_per_simd > 1.0) {
        // The same fragment-shaped loads with two or more workgroups per CU: they saturate the
        // vector memory path (a 512 x 1536 x 576 NT product runs 1.2-1.9 us faster on LDS panels).
        util *= 0.75;
    }
    const double stage_us = std::max(floor, waves_per_simd * mfma_us / util);
    double us = 4.0 + per * stage_us;
    // The reduction launch (its own latency floor) and the partials' round trip through HBM. At
    // 512 x 576 x 3072 the unsplit direct tile beats split-K 4 with its reduce by about 1 us.
    if (splits > 1) us += 7.5 + 2.0 * splits * d->batch * d->m * d->n * 4.0 / 5.0e6;
    return us;
}

int plan(const pxk_gemm_desc* d, Plan* p) {
    if (d->m <= 0 || d->n <= 0 || d->batch <= 0) return fail(PXK_ERR_INVALID, "pxk_gemm: m, n and batch must be positive");
    if (d->k < 0 || d->inner <= 0 || d->kgroups <= 0 || d->batch % d->inner != 0)
        return fail(PXK_ERR_INVALID, "pxk_gemm: bad k, inner or kgroups (batch must be a multiple of inner)");
    if (d->causal < 0 || d->causal > 3) return fail(PXK_ERR_INVALID, "pxk_gemm: unknown causal mode %d", d->causal);
    const int want = d->tile == 0 ? -1 : plan_tile(d->tile);  // the forced plan tile, if any
    if (d->tile != 0 && want < 0) return fail(PXK_ERR_INVALID, "pxk_gemm: unknown tile %d", d->tile);
    const TileInfo* forced = want >= 0 && want < kTiles ? &kTileInfo[want] : nullptr;
    if (d->splits < 0 || d->splits > 4096) return fail(PXK_ERR_INVALID, "pxk_gemm: bad split count %d", d->splits);
    p->e = find_entry(d->trans_a != 0, d->trans_b != 0, d->prologue, d->epilogue);
    if (!p->e)
        return fail(PXK_ERR_INVALID, "pxk_gemm: combination trans_a=%d trans_b=%d prologue=%d epilogue=%d is not built",
                    d->trans_a, d->trans_b, d->prologue, d->epilogue);
    if (d->a.ptr == nullptr || d->b.ptr == nullptr) return fail(PXK_ERR_INVALID, "pxk_gemm: A and B are required");
    // Outputs and inputs each epilogue needs.
    const int epi = d->epilogue;
    const bool need_c = !(epi == PXK_EPI_ROPE_REL || epi == PXK_EPI_VALUE_REL);
    if (need_c && d->c.ptr == nullptr) return fail(PXK_ERR_INVALID, "pxk_gemm: output C is required");
    if ((epi == PXK_EPI_ADD_RESID) && (d->c3.ptr == nullptr || d->x.ptr == nullptr))
        return fail(PXK_ERR_INVALID, "pxk_gemm: ADD_RESID needs C3 and X");
    if ((epi == PXK_EPI_ADD_RESID || epi == PXK_EPI_STORE_BIAS) && d->e_bias.ptr && d->c2.ptr == nullptr)
        return fail(PXK_ERR_INVALID, "pxk_gemm: a bias needs output C2");
    if ((epi == PXK_EPI_MUL_X || epi == PXK_EPI_SPV || epi == PXK_EPI_ROPE_REL) && d->x.ptr == nullptr)
        return fail(PXK_ERR_INVALID, "pxk_gemm: epilogue %d needs X", epi);
    if (epi == PXK_EPI_SWIGLU_REL && (d->x.ptr == nullptr) != (d->y.ptr == nullptr || d->w.ptr == nullptr))
        return fail(PXK_ERR_INVALID, "pxk_gemm: SWIGLU_REL takes X, Y and W together, or none (recomputed from Z2, Z3)");
    if (epi == PXK_EPI_SWIGLU_REL && d->x.ptr == nullptr && (d->e_bias.ptr || d->e_bias2.ptr || d->gate_act < 0 ||
                                                              d->gate_act > 1))
        return fail(PXK_ERR_INVALID, "pxk_gemm: SWIGLU_REL recomputes its factors only without biases (gate_act 0 or 1)");
    if ((epi == PXK_EPI_ROPE_REL || epi == PXK_EPI_VALUE_REL) &&
        (d->y.ptr == nullptr || d->z.ptr == nullptr || d->c2.ptr == nullptr))
        return fail(PXK_ERR_INVALID, "pxk_gemm: epilogue %d needs Y, Z and C2", epi);
    if (epi == PXK_EPI_SWIGLU_REL && (d->c2.ptr == nullptr || d->z2.ptr == nullptr || d->z3.ptr == nullptr))
        return fail(PXK_ERR_INVALID, "pxk_gemm: SWIGLU_REL needs C2, Z2 and Z3");
    if (epi == PXK_EPI_MUL_X_SPLIT && (d->x.ptr == nullptr || d->c2.ptr == nullptr || d->w.ptr == nullptr ||
                                       d->z2.ptr == nullptr || d->z3.ptr == nullptr))
        return fail(PXK_ERR_INVALID, "pxk_gemm: MUL_X_SPLIT needs X, C2, W, Z2 and Z3");
    if ((d->c2_den.ptr != nullptr || d->c2_den_bias.ptr != nullptr) &&
        (epi != PXK_EPI_MUL_X_SPLIT || d->c2_den.ptr == nullptr))
        return fail(PXK_ERR_INVALID, "pxk_gemm: c2_den (and its bias) belong to MUL_X_SPLIT, the bias only with c2_den");
    if (d->prologue == PXK_PRO_RMS &&
        (d->trans_a != 0 || d->kgroups != 1 || d->causal != PXK_CAUSAL_NONE || d->splits > 1 ||
         d->z.ptr != nullptr || d->z_bias.ptr != nullptr || d->k <= 0 || !(d->norm_eps >= 0.0f)))
        return fail(PXK_ERR_INVALID,
                    "pxk_gemm: the RMS prologue takes an untransposed A without k-groups, causal range or split-K, "
                    "gamma folded into B (no z or z_bias), k > 0 and norm_eps >= 0");
    if ((d->x_rms != nullptr) != (d->x_gamma != nullptr) ||
        (d->x_rms && ((epi != PXK_EPI_MUL_X && epi != PXK_EPI_MUL_X_SPLIT) || d->batch != 1)))
        return fail(PXK_ERR_INVALID, "pxk_gemm: x_rms and x_gamma go together, on an unbatched MUL_X or MUL_X_SPLIT");
    if (d->prologue == PXK_PRO_DIV_STAB && d->z.ptr == nullptr)
        return fail(PXK_ERR_INVALID, "pxk_gemm: the DIV_STAB prologue needs Z");
    if (d->prologue == PXK_PRO_DIV_STAB && (epi == PXK_EPI_ROPE_REL || epi == PXK_EPI_VALUE_REL))
        return fail(PXK_ERR_INVALID, "pxk_gemm: epilogue %d reads Z, which the DIV_STAB prologue owns", epi);
    if (epi == PXK_EPI_SWIGLU_FWD) {
        if (d->n % 64 != 0 || d->c2.ptr == nullptr || d->c3.ptr == nullptr || d->e_bias.ptr != nullptr)
            return fail(PXK_ERR_INVALID, "pxk_gemm: SWIGLU_FWD needs n a multiple of 64, C2 and C3, and no bias");
        if (forced && forced->bn % 64 != 0)
            return fail(PXK_ERR_INVALID, "pxk_gemm: SWIGLU_FWD needs 64-wide tile multiples (tile %d)", d->tile);
    }
    if (epi == PXK_EPI_ROPE_FWD) {
        const int64_t D = d->head_dim;
        if (D <= 0 || D % 2 != 0 || d->cos_t == nullptr || d->sin_t == nullptr || d->c3.ptr == nullptr)
            return fail(PXK_ERR_INVALID, "pxk_gemm: ROPE_FWD needs an even head_dim, cos/sin tables and C3");
        if (d->rope_cols < 0 || d->rope_cols > d->n || d->rope_cols % D != 0 || d->n % D != 0)
            return fail(PXK_ERR_INVALID, "pxk_gemm: ROPE_FWD rotates whole heads: rope_cols and n multiples of head_dim");
        if (!rope_fits(d, 128))
            return fail(PXK_ERR_INVALID, "pxk_gemm: ROPE_FWD needs whole heads inside a 128-wide tile");
        if (forced && !rope_fits(d, forced->bn))
            return fail(PXK_ERR_INVALID, "pxk_gemm: ROPE_FWD heads do not fit tile %d", d->tile);
    }
    if (epi == PXK_EPI_ROPE_REL) {
        const int64_t D = d->head_dim;
        if (D <= 0 || D % 2 != 0 || d->cos_t == nullptr || d->sin_t == nullptr)
            return fail(PXK_ERR_INVALID, "pxk_gemm: ROPE_REL needs an even head_dim and cos/sin tables");
        if (d->n % D != 0)
            return fail(PXK_ERR_INVALID, "pxk_gemm: ROPE_REL needs n to be a whole number of heads");
        if (!rope_fits(d, 128))
            return fail(PXK_ERR_INVALID, "pxk_gemm: ROPE_REL needs whole heads inside a 128-wide tile");
        if (forced && !rope_fits(d, forced->bn))
            return fail(PXK_ERR_INVALID, "pxk_gemm: ROPE_REL heads do not fit tile %d", d->tile);
    }
    if (d->k > (int64_t{1} << 40) || static_cast<double>(d->k) * d->kgroups / 32.0 > 2.0e9 || d->batch > (int64_t{1} << 31))
        return fail(PXK_ERR_INVALID, "pxk_gemm: k * kgroups or batch too large");

    // Up to 16 rows: the skinny kernels. NN: the widest column tile that still gives 160 workgroups
    // (64 columns for the SwiGLU gate, whose gate and up blocks interleave in 64s), and no split over
    // K unless a workgroup would stream more than 1 MiB of B.
    p->skinny = nullptr;
    if (d->tile == 0 || want == kSkinnyTile) {
        if (const SkinnyEntry* se = skinny_entry(d)) {
            p->skinny = se;
            p->tile = kSkinnyTile;
            p->tiles_m = 1;
            if (se->tb) {
                p->width = kSkinnyBN;
                p->splits = 1;
                p->kc = cdiv(d->k, 64) * 64;
            } else {
                p->width = 64;
                if (epi != PXK_EPI_SWIGLU_FWD)
                    while (p->width > 16 && cdiv(d->n, p->width) < 160) p->width /= 2;
                const int64_t s = d->splits > 0 ? d->splits : cdiv(d->k * p->width * 4, int64_t{1} << 20);
                p->kc = cdiv(cdiv(d->k, s), 16) * 16;
                p->splits = static_cast<int>(cdiv(d->k, p->kc));
            }
            p->tiles_n = cdiv(d->n, p->width);
            if (p->tiles_n * p->splits > (int64_t{1} << 31) - 1) return fail(PXK_ERR_INVALID, "pxk_gemm: grid too large");
            return PXK_OK;
        }
        if (want == kSkinnyTile)
            return fail(PXK_ERR_INVALID,
                        "pxk_gemm: the skinny tile needs m <= 16, batch 1, no prologue or causal range, A untransposed "
                        "and a built epilogue (STORE, STORE_BIAS, ADD_RESID, SWIGLU_FWD; NT: STORE, K up to the LDS)");
    }
    p->kc = 0;

    // Tile shape and split count: the forced ones, else the cheapest by estimate().
    int best_t = -1, best_s = 1;
    double best = 0.0;
    for (int t = 0; t < kTiles; ++t) {
        if (d->tile > 0 && t != want) continue;
        const TileInfo& ti = kTileInfo[t];
        if ((epi == PXK_EPI_ROPE_REL || epi == PXK_EPI_ROPE_FWD) && !rope_fits(d, ti.bn)) continue;
        if (epi == PXK_EPI_SWIGLU_FWD && ti.bn % 64 != 0) continue;
        const double stages = max_stages(d, ti.bm, ti.bk);
        const double tiles = static_cast<double>(live_tiles(d, ti.bm, ti.bn));
        // The 128x128 tile only pays off when its tiles alone fill the chip, unless it is the only
        // one that holds whole heads for a RoPE epilogue.
        const bool rope_epi = epi == PXK_EPI_ROPE_REL || epi == PXK_EPI_ROPE_FWD;
        const bool big_only = d->tile == 0 && t == 0 && !(rope_epi && !rope_fits(d, 64));
        if (big_only && tiles < 256.0) continue;
        for (int s = 1; s <= 64; s *= 2) {
            if (d->splits > 0 && s != 1) break;
            if (d->prologue == PXK_PRO_RMS && s != 1) break;  // the rows' sums of squares need the whole K
            const int splits = d->splits > 0 ? d->splits : s;
            if (d->splits == 0 && s > 1 && (big_only || stages / s < 2.0)) break;
            const double us = estimate(d, ti, tiles, stages, splits);
            if (best_t < 0 || us < best) {
                best = us;
                best_t = t;
                best_s = splits;
            }
        }
    }
    if (best_t < 0) return fail(PXK_ERR_INVALID, "pxk_gemm: no tile shape fits this descriptor");
    const TileInfo& ti = kTileInfo[best_t];
    p->tile = best_t;
    p->splits = best_s;
    p->tiles_m = cdiv(d->m, ti.bm);
    p->tiles_n = cdiv(d->n, ti.bn);
    const int64_t blocks = p->tiles_m * p->tiles_n * d->batch * p->splits;
    if (blocks > (int64_t{1} << 31) - 1) return fail(PXK_ERR_INVALID, "pxk_gemm: grid too large");
    return PXK_OK;
}

// M-tiles per group of the tile order (tile_of) when each XCD takes a run of `run` consecutive
// tiles: the divisor of tiles_m whose group_m x ceil(run / group_m) block of tiles reads the fewest
// panel bytes per XCD (group_m A panels of bm rows, the N-tiles' B panels of bn columns; K is
// common). With runs as long as a whole slice the order stays M-fastest (group_m = tiles_m). At 512
// x 576 on 32x48 tiles (16 x 12 tiles, runs of 24) that is 8 x 3 blocks, each A panel fetched by 4
// XCDs and each B panel by 2, against every XCD fetching every A panel in the M-fastest order.
int group_m(int64_t tiles_m, int64_t tiles_n, int64_t run, int bm, int bn) {
    if (run >= tiles_m * tiles_n) return static_cast<int>(tiles_m);
    int64_t best = tiles_m, best_cost = -1;
    for (int64_t gm = 1; gm <= tiles_m; ++gm) {
        if (tiles_m % gm != 0) continue;
        const int64_t cost = gm * bm + cdiv(run, gm) * bn;
        if (best_cost < 0 || cost < best_cost) {
            best_cost = cost;
            best = gm;
        }
    }
    return static_cast<int>(best);
}

size_t workspace_bytes(const pxk_gemm_desc* d, const Plan& p) {
    return p.splits > 1 ? static_cast<size_t>(p.splits) * d->batch * d->m * d->n * sizeof(float) : 0;
}

}  // namespace
}  // namespace pxk

using namespace pxk;

extern "C" int pxk_gemm_supported(int ta, int tb, int pro, int epi) { return find_entry(ta != 0, tb != 0, pro, epi) != nullptr; }

extern "C" int pxk_gemm_plan(const pxk_gemm_desc* d, int32_t* tile, int32_t* splits) {
    Plan p;
    if (const int rc = plan(d, &p)) return rc;
    if (tile) *tile = public_tile(p.tile);
    if (splits) *splits = p.splits;
    return PXK_OK;
}

extern "C" size_t pxk_gemm_workspace(const pxk_gemm_desc* d) {
    Plan p;
    if (plan(d, &p) != PXK_OK) return 0;
    return workspace_bytes(d, p);
}

extern "C" int pxk_gemm(const pxk_gemm_desc* d, void* stream) {
    if (d->m == 0 || d->n == 0 || d->batch == 0) return PXK_OK;
    Plan p;
    if (const int rc = plan(d, &p)) return rc;
    if (p.splits > 1) {
        const size_t need = workspace_bytes(d, p);
        if (d->workspace == nullptr || d->workspace_bytes < need || !aligned16(d->workspace)) {
            if (d->splits > 1)
                return fail(PXK_ERR_WORKSPACE, "pxk_gemm: split-K %d needs %zu workspace bytes (16-byte aligned)",
                            p.splits, need);
            // Library-chosen split without a workspace: the best single-pass plan instead.
            pxk_gemm_desc one = *d;
            one.splits = 1;
            if (const int rc = plan(&one, &p)) return rc;
        }
    }
    Args g{};
    g.M = d->m;
    g.N = d->n;
    g.K = d->k;
    g.batch = d->batch;
    g.inner = d->inner;
    g.kgroups = d->kgroups;
    g.causal = d->causal;
    g.splits = p.splits;
    g.beta = d->beta;
    g.eps = d->eps;
    g.a = to_op(d->a);
    g.b = to_op(d->b);
    g.c = to_op(d->c);
    g.z = to_op(d->z);
    g.zb = to_op(d->z_bias);
    g.c2 = to_op(d->c2);
    g.c3 = to_op(d->c3);
    g.x = to_op(d->x);
    g.y = to_op(d->y);
    g.w = to_op(d->w);
    g.z2 = to_op(d->z2);
    g.z3 = to_op(d->z3);
    g.eb = to_op(d->e_bias);
    g.eb2 = to_op(d->e_bias2);
    g.c2d = to_op(d->c2_den);
    g.c2db = to_op(d->c2_den_bias);
    g.xr = d->x_rms;
    g.xg = d->x_gamma;
    g.row_rms = d->prologue == PXK_PRO_RMS ? d->row_rms : nullptr;
    g.norm_eps = d->norm_eps;
    g.cos_t = d->cos_t;
    g.sin_t = d->sin_t;
    g.head_dim = d->head_dim;
    g.rope_half = d->rope_half;
    g.rope_cols = d->rope_cols;
    g.gate_act = d->gate_act;
    g.ws = d->workspace;
    // 128-bit loads when every base, stride and the contiguous extent allow them; the causal
    // K ranges start at multiples of the tile height, so they keep the alignment.
    const int64_t a_ext = d->trans_a ? d->m : d->k, b_ext = d->trans_b ? d->k : d->n;
    g.vec_a = vec_ok(d->a, a_ext) && (d->prologue == PXK_PRO_NONE || (vec_ok(d->z, a_ext) && vec_ok(d->z_bias, a_ext)));
    g.vec_b = vec_ok(d->b, b_ext);
    g.vec_e = d->n % 4 == 0 && vec_ok(d->c, d->n) && vec_ok(d->c2, d->n) && vec_ok(d->c3, d->n) &&
              vec_ok(d->x, d->n) && vec_ok(d->y, d->n) && vec_ok(d->w, d->n) && vec_ok(d->z2, d->n) &&
              vec_ok(d->z3, d->n) && vec_ok(d->e_bias, d->n) && vec_ok(d->e_bias2, d->n) &&
              vec_ok(d->c2_den, d->n) && vec_ok(d->c2_den_bias, d->n) &&
              (d->x_gamma == nullptr || aligned16(d->x_gamma)) &&
              (d->epilogue == PXK_EPI_ROPE_REL || d->epilogue == PXK_EPI_VALUE_REL ? vec_ok(d->z, d->n) : true);
    g.tiles_m = static_cast<int>(p.tiles_m);
    g.tiles_n = static_cast<int>(p.tiles_n);
    g.kc = p.kc;
    if (p.skinny) {
        const int mi = d->m <= 4 ? 0 : (d->m <= 8 ? 1 : 2);
        const int wi = p.width == 64 ? 0 : (p.width == 32 ? 1 : 2);
        g.bm = 16;
        const size_t lds = p.skinny->tb ? skinny_nt_lds(d) : 0;
        PXK_LAUNCH(p.skinny->k[mi][p.skinny->tb ? 0 : wi], dim3(static_cast<unsigned>(p.tiles_n * p.splits)),
                           dim3(NT), lds, S(stream), g);
        if (const int rc = launched("pxk_gemm (skinny)")) return rc;
        if (p.splits > 1) {
            const dim3 rgrid(static_cast<unsigned>(p.tiles_n), 1, 1);  // at least 16 rows per reduce workgroup
            PXK_LAUNCH(p.skinny->r[wi], rgrid, dim3(NT), 0, S(stream), g);
            return launched("pxk_gemm (skinny split-K reduce)");
        }
        return PXK_OK;
    }
    g.bm = kTileInfo[p.tile].bm;
    const int64_t blocks = p.tiles_m * p.tiles_n * d->batch * p.splits;
    g.remap = blocks % 8 == 0;
    g.group_m = g.remap ? group_m(p.tiles_m, p.tiles_n, blocks / 8, kTileInfo[p.tile].bm, kTileInfo[p.tile].bn)
                        : g.tiles_m;
    const int has_bias = d->prologue == PXK_PRO_DIV_STAB && d->z_bias.ptr != nullptr;
    PXK_LAUNCH(p.e->k[has_bias][p.tile], dim3(static_cast<unsigned>(blocks)),
                       dim3(static_cast<unsigned>(kTileInfo[p.tile].threads)), 0, S(stream), g);
    if (const int rc = launched("pxk_gemm")) return rc;
    if (p.splits > 1) {
        const int bn = kTileInfo[p.tile].bn;
        const int rs = 4 * NT / bn;
        const dim3 rgrid(static_cast<unsigned>(p.tiles_n), static_cast<unsigned>(cdiv(d->m, rs)),
                         static_cast<unsigned>(d->batch));
        if (rgrid.y > 65535 || rgrid.z > 65535) return fail(PXK_ERR_INVALID, "pxk_gemm: reduce grid too large");
        PXK_LAUNCH(p.e->r[p.tile], rgrid, dim3(NT), 0, S(stream), g);
        return launched("pxk_gemm split-K reduce");
    }
    return PXK_OK;
}

// ---- the allocation-free variant ------------------------------------------------------------------
// Split-K partials in a file-scope device array instead of a caller's workspace. Each GPU the library
// runs on holds its own copy of the array (PXK_GEMM_SCRATCH_BYTES) until the process ends. Its
// device address is looked up once per device with hipGetSymbolAddress: in host code the array's
// name is only a host-side stand-in, never a device address.
static __device__ __align__(256) float scratch[PXK_GEMM_SCRATCH_BYTES / sizeof(float)];

namespace pxk {
namespace {

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch[kScratchDevices] = {};

// The current device's copy of `scratch`, looked up on its first use on that device. That first use
// must not be inside a stream capture: the lookup is a runtime call, not stream work, so it is
// refused there (one eager call on the device first makes every later captured call valid).
int scratch_ptr(float** out, void* stream) {
    int dev = -1;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(PXK_ERR_LAUNCH, "pxk_gemm_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kScratchDevices) return fail(PXK_ERR_INVALID, "pxk_gemm_noalloc: device %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch[dev] == nullptr) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        const hipError_t q = hipStreamIsCapturing(S(stream), &cs);
        if (q != hipSuccess || cs != hipStreamCaptureStatusNone)
            return fail(PXK_ERR_INVALID,
                        "pxk_gemm_noalloc: the first split-K call on device %d is inside a stream capture; call it "
                        "once outside any capture first (the scratch address is looked up then)",
                        dev);
        void* p = nullptr;
        const hipError_t r = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (r != hipSuccess || p == nullptr)
            return fail(PXK_ERR_LAUNCH, "pxk_gemm_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                        hipGetErrorString(r));
        g_scratch[dev] = static_cast<float*>(p);
    }
    *out = g_scratch[dev];
    return PXK_OK;
}

}  // namespace
}  // namespace pxk

extern "C" int pxk_gemm_noalloc(const pxk_gemm_desc* d, void* stream) {
    if (d == nullptr) return fail(PXK_ERR_INVALID, "pxk_gemm_noalloc: descriptor is NULL");
    if (d->m == 0 || d->n == 0 || d->batch == 0) return PXK_OK;
    Plan p;
    if (const int rc = plan(d, &p)) return rc;
    const size_t need = workspace_bytes(d, p);
    if (need > PXK_GEMM_SCRATCH_BYTES)
        return fail(PXK_ERR_WORKSPACE,
                    "pxk_gemm_noalloc: split-K %d needs %zu bytes of partials, above the %zu-byte static scratch "
                    "(request fewer splits, or call pxk_gemm with a workspace)",
                    p.splits, need, static_cast<size_t>(PXK_GEMM_SCRATCH_BYTES));
    pxk_gemm_desc e = *d;
    e.workspace = nullptr;
    e.workspace_bytes = 0;
    if (need > 0) {
        if (const int rc = scratch_ptr(&e.workspace, stream)) return rc;
        e.workspace_bytes = PXK_GEMM_SCRATCH_BYTES;  // the plan does not depend on the workspace: pxk_gemm
    }                                                // recomputes the one checked above
    return pxk_gemm(&e, stream);
}

extern "C" int pxk_gemm_ex(const float* a, int ta, const float* b, int tb, float* out, int64_t m, int64_t k, int64_t n,
                           float beta, float* workspace, size_t workspace_bytes, void* stream) {
    if (m == 0 || n == 0) return PXK_OK;
    pxk_gemm_desc d;
    std::memset(&d, 0, sizeof(d));
    d.m = m;
    d.n = n;
    d.k = k;
    d.batch = d.inner = d.kgroups = 1;
    d.trans_a = ta;
    d.trans_b = tb;
    d.epilogue = PXK_EPI_STORE;
    d.beta = beta;
    d.a = pxk_operand{a, ta ? m : k, 0, 0, 0, 0};
    d.b = pxk_operand{b, tb ? k : n, 0, 0, 0, 0};
    d.c = pxk_operand{out, n, 0, 0, 0, 0};
    d.workspace = workspace;
    d.workspace_bytes = workspace_bytes;
    return pxk_gemm(&d, stream);
}
