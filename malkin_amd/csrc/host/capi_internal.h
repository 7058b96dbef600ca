// The C ABI's opaque handles (include/malkin_model.h, malkin_engine.h), shared by the translation units that
// implement them.
#pragma once

#include <memory>

#include "engine.h"
#include "gguf.h"
#include "model.h"

struct mk_model {
  std::unique_ptr<malkin_hip::GgufFile> file;
  std::unique_ptr<malkin_hip::Model> model;
};

struct mk_engine {
  std::unique_ptr<malkin_hip::Engine> engine;
  bool serving = false;  // an HTTP server owns the engine's loop (mk_server_start .. mk_server_stop)
};
