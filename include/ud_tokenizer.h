/*
 * ud_tokenizer.h -- SentencePiece detokenizer: token ids -> UTF-8 text.
 *
 * Replaces SentencePieceDecoder (Sources/DictatorCore/Decoding/SentencePiece.swift:5-31), which
 * NemotronStreamer uses for its transcript (Sources/DictatorCore/Nemotron/NemotronStreamer.swift:
 * 19, 48, 162).  Host code only (no device memory, no HIP calls); a loaded tokenizer is read-only
 * and may be shared by threads.
 *
 * Vocabulary (SentencePiece.swift:8-13): the text of `tokenizer.vocab`, one "piece<TAB>score" per
 * line, id = index among the non-empty lines.  A line ends at a '\n' that is not preceded by
 * '\r' (Swift splits Characters, and "\r\n" is one Character); its piece is the first non-empty
 * field between tabs (the whole line when it has no tab, "" when it is all tabs).
 *
 * Decoding (SentencePiece.swift:17-30): ids outside [0, size) are skipped; a byte-fallback piece
 * "<0xHH>" (two hex digits) contributes the byte 0xHH; "<unk>", "<s>", "</s>" and "<pad>"
 * contribute nothing; any other piece contributes its UTF-8 bytes with every U+2581 ("▁")
 * replaced by a space.  The bytes are then read as UTF-8 with each maximal ill-formed subpart
 * replaced by U+FFFD (Unicode's recommended practice, which Swift's String(decoding:as:) follows),
 * and one leading space is dropped.
 *
 * Differences from the Swift decoder, on inputs a SentencePiece vocabulary does not contain:
 * a byte piece with a sign ("<0x+A>", which Swift's integer parser would accept) is an ordinary
 * piece here; a "▁" followed by a combining mark inside a piece is replaced here, where Foundation's
 * non-literal search would leave it.
 *
 * Conventions as in ud_encoder.h (0 or a negative ud_status, ud_last_error()).
 */
#ifndef UD_TOKENIZER_H
#define UD_TOKENIZER_H

#include <stdint.h>

#include "ud_encoder.h"
#include "ud_streamer.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ud_tokenizer ud_tokenizer;

/* SentencePieceDecoder.init(vocabFile:) (SentencePiece.swift:8-13): reads and parses the file;
 * UD_ERR_INVALID when it cannot be read or is not UTF-8 (where the Swift initializer throws). */
UD_API int ud_tokenizer_load(const char* vocab_path, ud_tokenizer** out);
/* The same from the file's bytes already in memory (bytes need not be NUL-terminated). */
UD_API int ud_tokenizer_parse(const char* text, int64_t bytes, ud_tokenizer** out);
UD_API void ud_tokenizer_destroy(ud_tokenizer* t);
/* SentencePieceDecoder.count (SentencePiece.swift:15). */
UD_API int ud_tokenizer_size(const ud_tokenizer* t, int32_t* size);
/* Piece `id` as UTF-8 bytes: the first cap of them into out; *len receives the total. */
UD_API int ud_tokenizer_piece(const ud_tokenizer* t, int32_t id, char* out, int64_t cap, int64_t* len);
/* SentencePieceDecoder.decode (SentencePiece.swift:17-30): the text of ids[0 .. n) as UTF-8.  The
 * first cap bytes go to out (no terminating NUL); *len receives the text's full length, so a call
 * with cap 0 sizes the buffer. */
UD_API int ud_tokenizer_decode(const ud_tokenizer* t, const int32_t* ids, int32_t n, char* out, int64_t cap,
                               int64_t* len);

/* NemotronStreamer.text (NemotronStreamer.swift:48): the transcript of stream `id` so far, its
 * tokens (ud_streamer_tokens) decoded by t; out / cap / len as for ud_tokenizer_decode. */
UD_API int ud_streamer_text(const ud_streamer* s, int32_t id, const ud_tokenizer* t, char* out, int64_t cap,
                            int64_t* len);

#ifdef __cplusplus
}
#endif

#endif /* UD_TOKENIZER_H */
