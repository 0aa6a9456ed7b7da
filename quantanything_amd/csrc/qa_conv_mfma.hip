// int8 MFMA convolution / GEMM: tile choice and the variants with weights
// staged in LDS (kernel templates: qa_conv_mfma.h).
#include "qa_conv_mfma.h"

namespace qa {

bool mfma_launch_lds(const ConvArgs& b, int wm, bool split, int epi,
                     hipStream_t st) {
    return launch_variant<true>(b, wm, split, epi, st);
}

// The launch form of a descriptor's arguments: whether the output (and
// residual / copy) is dense channels-last (fastio, pixel strides *_pst),
// the table epilogue when a plan applies, and the magic divisors of the
// tap decode. Returns the epilogue variant (epi when no plan applies).
int fast_io_args(const ConvArgs& a, ConvArgs& b, int epi) {
    b = a;
    // dense channels-last int8 output (and residual / copy): 4-channel
    // words of a pixel at pixel * sp + channel, 4-byte aligned
    {
        const int64_t ohw = (int64_t)a.OH * a.OW;
        // pixel stride: sp, or the row stride sn of a GEMM (one pixel a row)
        auto pst = [&](int64_t sn, int64_t sp) { return ohw == 1 ? sn : sp; };
        auto dense = [&](const void* p, int64_t sn, int64_t sc, int64_t sp) {
            return p == nullptr ||
                   (sc == 1 && (ohw == 1 || sn == ohw * sp) &&
                    pst(sn, sp) % 4 == 0 && (uintptr_t)p % 4 == 0);
        };
        b.fastio = a.mode == EPI_QUANT && (a.G == 1 || a.Cog % 4 == 0) &&
                   dense(a.y, a.y_sn, a.y_sc, a.y_sp) &&
                   dense(a.res, a.res_sn, a.res_sc, a.res_sp) &&
                   dense(a.y2, a.y2_sn, a.y2_sc, a.y2_sp);
        b.y_pst = pst(a.y_sn, a.y_sp);
        b.res_pst = pst(a.res_sn, a.res_sp);
        b.y2_pst = pst(a.y2_sn, a.y2_sp);
    }
    if (a.mode == EPI_QUANT && a.plan && b.fastio) epi = Q8_TABLE;
    b.mg_cb = (((uint64_t)1 << 32) + a.CB - 1) / (uint64_t)a.CB;
    b.mg_kw = (((uint64_t)1 << 32) + a.KW - 1) / (uint64_t)a.KW;
    return epi;
}

// Tile choice (from measured sweeps over the channel-block width WM and
// K-splitting on MI355X): the widest channel block that still gives about
// 1.5 waves per SIMD (0.75 when K is long, >= 9 steps: those waves are long
// enough on their own), and the 4 waves of a work-group split K only when
// even 16-channel blocks leave most SIMDs idle.
bool launch_conv_mfma(const ConvArgs& a, hipStream_t st) {
    if (a.M <= 0 || a.Cog <= 0 || a.G <= 0) return true;
    if (a.M >= ((int64_t)1 << 31) || a.KGp < 4 || (a.KGp & 3) ||
        a.KGp >= (1 << 16) || a.CB < 1 || a.KW < 1 ||
        (int64_t)(a.KH - 1) * a.DH >= 32768 ||
        (int64_t)(a.KW - 1) * a.DW >= 32768) {
        set_error("launch_conv_mfma", "unsupported problem size");
        return false;
    }
    int epi = a.mode;
    if (a.mode == EPI_QUANT) {
        if (a.y_code != 1) {
            set_error("launch_conv_mfma", "int8 output expected");
            return false;
        }
        epi = Q8_GENERAL;  // chosen below, once the layout is known
    }
    ConvArgs b;
    epi = fast_io_args(a, b, epi);
    // bands of output rows with operands in LDS (tile hint bit 11, with
    // wm in the low bits)
    // (ignored, like every hint, where it does not apply)
    if ((a.tile_hint & TILE_VALID) && ((a.tile_hint >> 11) & 1)) {
        const int bw = a.tile_hint & 0xff;
        if ((bw == 1 || bw == 2 || bw == 4) && conv_band_applies(b, epi, bw))
            return launch_conv_band(b, bw, st);
    }
    // weights in registers, bands in LDS (tile hint bit 12, with wm in the
    // low bits); without a hint, the default for convolutions of more than
    // one 64-byte K-step (measured the fastest choice for most 3x3 layers)
    if ((a.tile_hint & TILE_VALID) && ((a.tile_hint >> 12) & 1)) {
        const int ww = a.tile_hint & 0xf;  // bits 4..7: the band height
        if (conv_wr_applies(b, epi, ww)) return launch_conv_wr(b, ww, st);
    }
    if (!(a.tile_hint & TILE_VALID) && a.KGp > 4 && (a.KH > 1 || a.KW > 1)) {
        for (int ww = a.Cog >= 64 ? 4 : a.Cog >= 32 ? 2 : 1; ww >= 1; ww >>= 1)
            if (conv_wr_applies(b, epi, ww)) return launch_conv_wr(b, ww, st);
    }
    // narrow GEMMs / pointwise convolutions, one 16 x 16 block a wave with
    // all of its operands in registers (tile hint bit 13)
    if ((a.tile_hint & TILE_VALID) && ((a.tile_hint >> 13) & 1) &&
        gemm_narrow_applies(b, epi))
        return launch_gemm_narrow(b, st, 1 + ((a.tile_hint >> 4) & 3));
    // large GEMMs: 128 x 128 blocks (tile hint bit 10 chooses; its low
    // bits 3 or 4 the direct-to-LDS pipeline with that many stages)
    if (gemm_big_applies(b, epi)) {
        bool big = a.M >= 1024 && a.Cout >= 128;
        int stages = 0;
        if (a.tile_hint & TILE_VALID) {
            big = (a.tile_hint >> 10) & 1;
            stages = a.tile_hint & 0xff;
        }
        if (big) return launch_gemm_big(b, st, stages);
    }
    const int64_t ntiles = ceil_div(a.M, 16);
    const int64_t simds = 4 * (int64_t)cu_count();
    auto waves = [&](int wm, bool split) {
        return ntiles * ceil_div(a.Cog, 16 * wm) * a.G * (split ? 4 : 1);
    };
    const int KS = a.KGp >> 2;
    const int wm_max =
        a.Cog <= 16 ? 1 : (a.Cog <= 32 ? 2 : (a.Cog <= 64 ? 4 : 8));
    const int64_t want = KS >= 9 ? simds * 3 / 4 : simds * 3 / 2;
    int wm = wm_max;
    while (wm > 1 && waves(wm, false) < want) wm >>= 1;
    bool split = a.layout == 0 && KS >= 4 && waves(wm, false) < simds / 2;
    // weights staged in LDS when they fit next to the tables (64 KB per
    // work-group), otherwise read from L2
    auto lds_limit = [&](int w) {
        return 65536 - 3072 - 64 - (split ? 3 * (w * 4 + 1) * 256 : 0);
    };
    auto fits = [&](int w) {
        return alds_bytes(w, a.KGp) + (a.layout == 0 ? a.KGp * 16 : 0) <=
                   lds_limit(w) &&
               (int64_t)w * 16 * a.KGp <= ALDS_CHUNKS;
    };
    bool alds = fits(wm);
    // a caller's measured choice (qa_conv_desc.tile), where it applies
    if (a.tile_hint & TILE_VALID) {
        const int hw = a.tile_hint & 0xff;
        if (hw >= 1 && hw <= wm_max && (hw & (hw - 1)) == 0) {
            wm = hw;
            split = ((a.tile_hint >> 8) & 1) && a.layout == 0;
            alds = ((a.tile_hint >> 9) & 1) && fits(wm);
        }
    }
    return alds ? mfma_launch_lds(b, wm, split, epi, st)
                : mfma_launch_l2(b, wm, split, epi, st);
}

}  // namespace qa
