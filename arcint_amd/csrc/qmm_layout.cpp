// qmm_layout.cpp - the weight image (host side): type table, image sizes and
// the placement of GGUF block bytes in tile-groups (see qmm_internal.h).
// Pure host code: the same functions serve qmm_tensor_set/get and the
// host-side pack/unpack entry points.
#include <algorithm>
#include <cstring>

#include "qmm_internal.h"
#include "qmm_layout.h"

namespace qmm {

namespace {

// type, blck, bytes, bpg, nchunk, tail, tg
constexpr TypeLayout kLayouts[] = {
    { QMM_TYPE_Q4_0,   32,  18,  8, 9,  0, tile_group_bytes(QMM_TYPE_Q4_0) },
    { QMM_TYPE_Q8_0,   32,  34,  8, 17, 0, tile_group_bytes(QMM_TYPE_Q8_0) },
    { QMM_TYPE_Q4_K,   256, 144, 1, 9,  0, tile_group_bytes(QMM_TYPE_Q4_K) },
    { QMM_TYPE_Q6_K,   256, 210, 1, 13, 2, tile_group_bytes(QMM_TYPE_Q6_K) },
    { QMM_TYPE_IQ4_XS, 256, 136, 1, 8,  8, tile_group_bytes(QMM_TYPE_IQ4_XS) },
    { QMM_TYPE_Q5_K,   256, 176, 1, 11, 0, tile_group_bytes(QMM_TYPE_Q5_K) },
    { QMM_TYPE_IQ4_NL, 32,  18,  8, 9,  0, tile_group_bytes(QMM_TYPE_IQ4_NL) },
};
// the planes fill the tile-group exactly
constexpr bool planes_fill(const TypeLayout & L) { return L.nchunk * kChunk + kTileRows * L.tail == L.tg; }
static_assert(planes_fill(kLayouts[0]) && planes_fill(kLayouts[1]) && planes_fill(kLayouts[2]) && planes_fill(kLayouts[3]) &&
                  planes_fill(kLayouts[4]) && planes_fill(kLayouts[5]) && planes_fill(kLayouts[6]),
              "chunk planes + tail plane = tile-group bytes");

}  // namespace

const TypeLayout * type_layout(int type) {
    for (const auto & L : kLayouts)
        if (L.type == type) return &L;
    return nullptr;
}

bool image_shape(const TypeLayout & L, const int64_t ne[4], ImageShape * s) {
    if (ne[0] <= 0 || ne[0] % L.blck || ne[1] <= 0 || ne[2] <= 0 || ne[3] <= 0) return false;
    s->K = ne[0];
    s->M = ne[1];
    s->nmat = ne[2] * ne[3];
    s->bpr = ne[0] / L.blck;
    s->G = (ne[0] + kGroupW - 1) / kGroupW;
    s->ntiles = (ne[1] + kTileRows - 1) / kTileRows;
    const size_t raw = (size_t)s->nmat * (size_t)s->ntiles * (size_t)s->G * (size_t)L.tg;
    s->bytes = (raw + 255) / 256 * 256;
    return true;
}

int block_pieces(const TypeLayout & L, Piece out[16]) {
    int n = 0;
    switch (L.type) {
        case QMM_TYPE_Q4_0:
        case QMM_TYPE_IQ4_NL:
            out[n++] = { 2, 16, 0, 16, kChunk };
            out[n++] = { 0, 2, 8 * kChunk, 16, 2 };
            break;
        case QMM_TYPE_Q8_0:
            out[n++] = { 2, 16, 0, 16, 2 * kChunk };
            out[n++] = { 18, 16, kChunk, 16, 2 * kChunk };
            out[n++] = { 0, 2, 16 * kChunk, 16, 2 };
            break;
        case QMM_TYPE_Q4_K:
            for (int c = 0; c < 8; ++c) out[n++] = { 16 + 16 * c, 16, c * kChunk, 16, 0 };
            out[n++] = { 0, 16, 8 * kChunk, 16, 0 };
            break;
        case QMM_TYPE_Q6_K:
            for (int c = 0; c < 8; ++c) out[n++] = { 16 * c, 16, c * kChunk, 16, 0 };
            for (int c = 0; c < 4; ++c) out[n++] = { 128 + 16 * c, 16, (8 + c) * kChunk, 16, 0 };
            out[n++] = { 192, 16, 12 * kChunk, 16, 0 };
            out[n++] = { 208, 2, 13 * kChunk, 2, 0 };
            break;
        case QMM_TYPE_Q5_K:
            for (int c = 0; c < 8; ++c) out[n++] = { 48 + 16 * c, 16, c * kChunk, 16, 0 };
            out[n++] = { 0, 16, 8 * kChunk, 16, 0 };
            out[n++] = { 16, 16, 9 * kChunk, 16, 0 };
            out[n++] = { 32, 16, 10 * kChunk, 16, 0 };
            break;
        case QMM_TYPE_IQ4_XS:
            for (int c = 0; c < 8; ++c) out[n++] = { 8 + 16 * c, 16, c * kChunk, 16, 0 };
            out[n++] = { 0, 8, 8 * kChunk, 8, 0 };
            break;
        default: break;
    }
    return n;
}

// global tile of global row R (R = mat * M + m)
int64_t tile_of_row(const ImageShape & s, int64_t R) { return (R / s.M) * s.ntiles + (R % s.M) / kTileRows; }

// first global row of global tile T and one past its last row
void tile_rows(const ImageShape & s, int64_t T, int64_t * r0, int64_t * r1) {
    const int64_t mat = T / s.ntiles, t = T % s.ntiles;
    *r0 = mat * s.M + t * kTileRows;
    *r1 = mat * s.M + std::min<int64_t>(s.M, (t + 1) * kTileRows);
}

// byte offset of (block slot p of group g of row r) in the image of global
// tiles starting at T0, for global tile T
static inline size_t tg_off(const TypeLayout & L, const ImageShape & s, int64_t T, int64_t T0, int64_t g) {
    return (size_t)((T - T0) * s.G + g) * (size_t)L.tg;
}

void pack_blocks(const TypeLayout & L, const ImageShape & s, const uint8_t * src, int64_t b0, int64_t nb,
                 uint8_t * img, int64_t T0) {
    Piece pc[16];
    const int np = block_pieces(L, pc);
    for (int64_t i = 0; i < nb; ++i) {
        const int64_t b = b0 + i, R = b / s.bpr, kb = b % s.bpr;
        const int64_t T = tile_of_row(s, R);
        const int r = (int)((R % s.M) % kTileRows);
        const int64_t g = kb / L.bpg;
        const int p = (int)(kb % L.bpg);
        uint8_t * tgp = img + tg_off(L, s, T, T0, g);
        const uint8_t * blk = src + (size_t)i * L.bytes;
        for (int q = 0; q < np; ++q)
            memcpy(tgp + pc[q].dst + r * pc[q].row_step + p * pc[q].slot_step, blk + pc[q].src, (size_t)pc[q].size);
    }
}

void unpack_blocks(const TypeLayout & L, const ImageShape & s, const uint8_t * img, int64_t T0, int64_t b0, int64_t nb,
                   uint8_t * dst) {
    Piece pc[16];
    const int np = block_pieces(L, pc);
    for (int64_t i = 0; i < nb; ++i) {
        const int64_t b = b0 + i, R = b / s.bpr, kb = b % s.bpr;
        const int64_t T = tile_of_row(s, R);
        const int r = (int)((R % s.M) % kTileRows);
        const int64_t g = kb / L.bpg;
        const int p = (int)(kb % L.bpg);
        const uint8_t * tgp = img + tg_off(L, s, T, T0, g);
        uint8_t * blk = dst + (size_t)i * L.bytes;
        for (int q = 0; q < np; ++q)
            memcpy(blk + pc[q].src, tgp + pc[q].dst + r * pc[q].row_step + p * pc[q].slot_step, (size_t)pc[q].size);
    }
}

void zero_row_padding(const TypeLayout & L, const ImageShape & s, int64_t R, uint8_t * img, int64_t T0) {
    const int64_t nslots = s.G * L.bpg;
    if (nslots == s.bpr) return;
    Piece pc[16];
    const int np = block_pieces(L, pc);
    const int64_t T = tile_of_row(s, R);
    const int r = (int)((R % s.M) % kTileRows);
    for (int64_t kb = s.bpr; kb < nslots; ++kb) {
        uint8_t * tgp = img + tg_off(L, s, T, T0, kb / L.bpg);
        const int p = (int)(kb % L.bpg);
        for (int q = 0; q < np; ++q) memset(tgp + pc[q].dst + r * pc[q].row_step + p * pc[q].slot_step, 0, (size_t)pc[q].size);
    }
}

}  // namespace qmm
