// handles.hpp -- the C surface's opaque handles, shared by the host mirror's
// translation units (the aligner composes an encoder and a decoder).
#pragma once

#include "audio_encoder.hpp"
#include "decoder_prefill.hpp"

struct qah_tdec {
  qa_host::TextDecoder* d;
};

struct qah_aenc {
  qa_host::AudioEncoder* e;
};
