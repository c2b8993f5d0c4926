// ref_tok.cpp -- C entry points over the reference's own tokenizer headers
// (tensormark/bpe.h, tensormark/sp_tokenizer.h), compiled where they lie by
// oracle/Makefile into oracle/_ref/libtok_ref.so.  TEST INFRASTRUCTURE ONLY:
// the checker for tms_token_table_* (piece bytes of both tokenizer kinds).

#include <cstring>
#include <string>
#include <vector>

#include "bpe.h"
#include "sp_tokenizer.h"

extern "C" {

// tmbpe::unicode_str_to_bytes (bpe.h:91-110) on one piece: the byte count
// written, or -1 when the reference throws.
int ref_bpe_bytes(const char* piece, size_t len, char* out, size_t cap) {
    try {
        const std::string b = tmbpe::unicode_str_to_bytes(std::string(piece, len));
        if (b.size() > cap) return -1;
        std::memcpy(out, b.data(), b.size());
        return (int)b.size();
    } catch (...) {
        return -1;
    }
}

// tmspm::Tokenizer::build_bytes (sp_tokenizer.h:154-172) over n pieces,
// then piece_bytes(id) for every id, concatenated into out with per-id
// lengths in lens_out.  Returns the total, or -1 on a throw or overflow.
int ref_spm_bytes(const char* const* pieces, const size_t* lens, const unsigned char* types, int n,
                  char* out, size_t cap, int* lens_out) {
    try {
        tmspm::Tokenizer t;
        t.pieces.resize((size_t)n);
        for (int i = 0; i < n; ++i) {
            t.pieces[(size_t)i].piece.assign(pieces[i], lens[i]);
            t.pieces[(size_t)i].type = static_cast<tmspm::PieceType>(types[i]);
        }
        t.build_bytes();
        size_t at = 0;
        for (int i = 0; i < n; ++i) {
            const std::string& b = t.piece_bytes(i);
            if (at + b.size() > cap) return -1;
            std::memcpy(out + at, b.data(), b.size());
            at += b.size();
            lens_out[i] = (int)b.size();
        }
        return (int)at;
    } catch (...) {
        return -1;
    }
}

}  // extern "C"
