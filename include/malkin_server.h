/*
 * malkin-mi355x: C ABI of the HTTP API over the device engine (libmalkin_hip.so): the reference's OpenAI-style server
 * (src/server.cpp:193-209 routes, 315-358 /v1/completions) for a build without tokenizer, so prompts and
 * completions are token ids.
 *
 *   GET  /health          {"status":"ok"}
 *   GET  /v1/models       the one model: id, context_length
 *   POST /v1/completions  {"prompt": [ids], "max_tokens": 16, "temperature": .., "top_p": .., "top_k": ..,
 *                          "min_p": .., "presence_penalty": .., "frequency_penalty": .., "seed": ..,
 *                          "stop_token_ids": [ids], "stream": false}
 *                         -> choices[0].tokens (ids), finish_reason "stop" | "length", usage, timings; with
 *                            "stream": one server-sent event per engine step with the new ids, a final event with
 *                            the finish reason, then "data: [DONE]". A client that disconnects cancels its request.
 *   /v1/chat/completions, /v1/messages: 400 (they need a tokenizer and chat template).
 * Errors are {"error": {"message", "type"}} with status 400 (bad request, the engine's refusal texts), 404, 405,
 * 500 or 503 (no engine). Status codes and mk_last_error() as in malkin_hip.h.
 */
#ifndef MALKIN_SERVER_H
#define MALKIN_SERVER_H

#include "malkin_engine.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mk_server mk_server;

/* serve(engine, host, port) (server.cpp:481-495) without blocking: binds host:port (port 0: a free port, written to
   bound_port) and answers on background threads; one thread owns the engine's loop (the reference's worker), so
   the engine must not be driven through mk_engine_* until mk_server_stop. engine NULL: /health and /v1/models only
   (503 for completions). model_id: the name /v1/models reports. */
int mk_server_start(mk_engine* engine, const char* model_id, const char* host, int port, mk_server** out,
                    int* bound_port);
/* Stops accepting, cancels requests in flight (finish "cancelled"), waits for the connections, frees the server;
   the engine is usable again afterwards. */
int mk_server_stop(mk_server* server);

#ifdef __cplusplus
}
#endif

#endif
