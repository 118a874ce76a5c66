{-# LANGUAGE OverloadedStrings #-}
{-# LANGUAGE RecordWildCards #-}
{-# LANGUAGE ScopedTypeVariables #-}

{-|
Module: Gemma.Model
Description: Gemma 3 decode on MI355X through libgemma_hip

The same exports and signatures as the reference's Gemma.Model
(src/Gemma/Model.hs:19-31), with the bodies of the model record, the loaders
and the inference calls replaced: the weights, the KV cache and every
kernel of the step live in libgemma_hip (Graphics.HIP) instead of Dawn
tensors and WGSL shaders.

Kept here, as in the reference, with no Dawn type in them: the config
record and its presets (src/Gemma/Model.hs:106-237) and configFromGGUF
(src/Gemma/Model.hs:843-902), which reads the file's metadata through the
reference's own Gemma.GGUF.

As in the reference, the device K/V belong to the model (one sequence per
model), and a KVCache value carries the lengths: its layer-0 cacheLen is
the position of the next step (src/Gemma/Model.hs:1332-1334).  A step on an
older KVCache value rewinds the device cache to that value's length
(gh_kv_truncate), so KVCache keeps the persistent-value meaning it has in
the reference.
-}
module Gemma.Model
  ( GemmaConfig(..)
  , GemmaModel(..)
  , gemma2_2BConfig
  , gemma1BConfig
  , gemma3_1BConfig
  , tinyGemmaConfig
  , loadGemmaModel
  , loadGemmaModelFromGGUF
  , configFromGGUF
  , runGemmaInference
  , runGemmaInferenceCached
  , runGemmaInferenceCachedWithLayer0
  ) where

import Control.Monad (forM_, when)
import Control.Monad.IO.Class (liftIO)
import Control.Monad.Trans.Cont (ContT)
import Data.Bits ((.|.))
import Data.Int (Int32)
import Data.Maybe (fromMaybe)
import qualified Data.Text as T
import qualified Data.Vector as BV
import qualified Data.Vector.Storable as V
import qualified Data.Vector.Storable.Mutable as VM
import Data.Vector.Storable (Vector)
import Foreign.C.String (withCString)
import Foreign.C.Types (CFloat)
import Foreign.ForeignPtr (withForeignPtr)
import Foreign.Marshal.Alloc (alloca)
import Foreign.Ptr (Ptr, castPtr, nullPtr)
import Foreign.Storable (peek, sizeOf)

import Gemma.KVCache (KVCache(..), LayerKVCache(..), cacheLength, initKVCache)
import qualified Gemma.GGUF as GGUF
import Gemma.SafeTensors (getTensor, hasTensor, loadSafeTensors)
import qualified Graphics.HIP as HIP
import Graphics.HIP (check)

-- | Hyper-parameters and feature flags (src/Gemma/Model.hs:106-129): the
-- reference's record, field for field, so callers that build or pattern
-- match a config compile unchanged.  gcUseFP16 / gcUseVec4 / gcUseFusion
-- selected WGSL shader variants and have no effect here (the HIP step
-- computes in f32 on Q4_0 or f32 weights); gcLocalRopeScaling,
-- gcGlobalRopeScaling and gcQueryHeadDimNormalize are carried as the
-- reference carries them (its step reads none of them).
data GemmaConfig = GemmaConfig
  { gcVocabSize :: Int
  , gcHiddenDim :: Int
  , gcNumLayers :: Int
  , gcNumHeads :: Int
  , gcNumKVHeads :: Int
  , gcHeadDim :: Int
  , gcFFNDim :: Int
  , gcRopeBase :: Float
  , gcUseFP16 :: Bool
  , gcUseVec4 :: Bool
  , gcUseFusion :: Bool
  , gcUseQKNorm :: Bool
  , gcUsePostAttnNorm :: Bool
  , gcUsePostFFNNorm :: Bool
  , gcUseSlidingWindow :: Bool
  , gcSlidingWindowSize :: Int
  , gcLocalRopeScaling :: Float
  , gcGlobalRopeScaling :: Float
  , gcQueryHeadDimNormalize :: Bool
  , gcUseZeroCenteredRMSNorm :: Bool
  } deriving (Show, Eq)

-- | The Gemma 1 / 2 layout: none of the Gemma 3 features, one RoPE base.
plainConfig :: Int -> Int -> Int -> Int -> Int -> Int -> Int -> GemmaConfig
plainConfig vocab hidden layers heads kvHeads headDim ffn = GemmaConfig
  { gcVocabSize = vocab, gcHiddenDim = hidden, gcNumLayers = layers, gcNumHeads = heads
  , gcNumKVHeads = kvHeads, gcHeadDim = headDim, gcFFNDim = ffn, gcRopeBase = 10000.0
  , gcUseFP16 = False, gcUseVec4 = False, gcUseFusion = False
  , gcUseQKNorm = False, gcUsePostAttnNorm = False, gcUsePostFFNNorm = False
  , gcUseSlidingWindow = False, gcSlidingWindowSize = 0
  , gcLocalRopeScaling = 1.0, gcGlobalRopeScaling = 1.0
  , gcQueryHeadDimNormalize = False, gcUseZeroCenteredRMSNorm = False
  }

-- | Gemma 1B (src/Gemma/Model.hs:131-156).
gemma1BConfig :: GemmaConfig
gemma1BConfig = plainConfig 256000 2048 24 16 8 128 5504

-- | Gemma 2 2B (src/Gemma/Model.hs:158-183).
gemma2_2BConfig :: GemmaConfig
gemma2_2BConfig = plainConfig 256000 2304 26 8 4 256 9216

-- | The reference's tiny synthetic test model (src/Gemma/Model.hs:185-210).
tinyGemmaConfig :: GemmaConfig
tinyGemmaConfig = plainConfig 1000 128 2 4 2 32 384

-- | Gemma 3 1B (src/Gemma/Model.hs:212-237): QK-norm, post-norms, a 512
-- window, zero-centred RMSNorm weights, RoPE base 1e6.
gemma3_1BConfig :: GemmaConfig
gemma3_1BConfig = (plainConfig 262144 1152 26 4 1 256 6912)
  { gcRopeBase = 1000000.0
  , gcUseQKNorm = True, gcUsePostAttnNorm = True, gcUsePostFFNNorm = True
  , gcUseSlidingWindow = True, gcSlidingWindowSize = 512
  , gcQueryHeadDimNormalize = True, gcUseZeroCenteredRMSNorm = True
  }

-- | configFromGGUF (src/Gemma/Model.hs:843-902): the gemma3.* metadata of a
-- parsed GGUF file with the Gemma 3 feature flags on.  The vocabulary is the
-- row count of token_embd.weight when the file has that tensor (what
-- gh_model_load_gguf uses, so this config and the loaded model agree), else
-- the length of tokenizer.ggml.tokens, else 256000; the window defaults to
-- 512.  A missing required key is an error, as in the reference.
configFromGGUF :: GGUF.GGUFFile -> GemmaConfig
configFromGGUF gf = gemma3_1BConfig
  { gcVocabSize = vocab
  , gcHiddenDim = int "gemma3.embedding_length"
  , gcNumLayers = int "gemma3.block_count"
  , gcNumHeads = int "gemma3.attention.head_count"
  , gcNumKVHeads = int "gemma3.attention.head_count_kv"
  , gcHeadDim = int "gemma3.attention.key_length"
  , gcFFNDim = int "gemma3.feed_forward_length"
  , gcRopeBase = req "gemma3.rope.freq_base" (GGUF.getMetadataFloat gf "gemma3.rope.freq_base")
  , gcSlidingWindowSize = maybe 512 fromIntegral (GGUF.getMetadataInt gf "gemma3.attention.sliding_window")
  }
  where
    req key = fromMaybe (error ("Missing or invalid metadata: " ++ T.unpack key))
    int key = fromIntegral (req key (GGUF.getMetadataInt gf key))
    vocab
      | GGUF.hasTensor gf "token_embd.weight" = case GGUF.getTensorShape gf "token_embd.weight" of
          [_, rows] -> fromIntegral rows
          _ -> error "token_embd.weight is not a matrix"
      | otherwise = case GGUF.getMetadata gf "tokenizer.ggml.tokens" of
          Just (GGUF.MetaArray toks) -> length toks
          _ -> 256000

-- | The model: config plus library handles.  (The reference's record holds
-- Dawn Context / Tensor / KernelCode fields, src/Gemma/Model.hs:243-257.)
data GemmaModel dtype = GemmaModel
  { gmConfig  :: GemmaConfig
  , gmContext :: HIP.Context   -- ^ device and stream
  , gmHandle  :: HIP.Model     -- ^ weights on the device (Q4_0 repacked or f32)
  , gmCache   :: HIP.Cache     -- ^ the model's device K/V
  , gmMaxSeq  :: Int           -- ^ positions the device cache holds
  }

-- | The reference's cache capacity (src/Gemma/Model.hs:481).
defaultMaxSeq :: Int
defaultMaxSeq = 2048

-- | GemmaConfig -> gh_config.  The reference's arithmetic (one RoPE base,
-- gcRopeBase, on every layer; the sliding window as a prefix of the cache:
-- quirks of src/Gemma/Model.hs:486 and TransformerBlockGPU.hs:238-240) is
-- GH_MODE_REF, so the drop-in reproduces the reference's outputs.
toGh :: GemmaConfig -> Int -> HIP.GhConfig
toGh GemmaConfig{..} maxSeq = HIP.GhConfig
  { HIP.ghVocab = i gcVocabSize, HIP.ghHidden = i gcHiddenDim, HIP.ghLayers = i gcNumLayers
  , HIP.ghHeads = i gcNumHeads, HIP.ghKVHeads = i gcNumKVHeads, HIP.ghHeadDim = i gcHeadDim
  , HIP.ghFFN = i gcFFNDim, HIP.ghMaxSeq = i maxSeq
  , HIP.ghSlidingWindow = if gcUseSlidingWindow then i gcSlidingWindowSize else 0
  , HIP.ghGlobalEvery = 0
  , HIP.ghThetaLocal = gcRopeBase, HIP.ghThetaGlobal = gcRopeBase, HIP.ghRmsEps = 1.0e-6
  , HIP.ghMode = HIP.modeRef
  , HIP.ghFlags = flag gcUseQKNorm HIP.flagQKNorm .|. flag gcUsePostAttnNorm HIP.flagPostAttnNorm
                  .|. flag gcUsePostFFNNorm HIP.flagPostFFNNorm .|. flag gcUseZeroCenteredRMSNorm HIP.flagZeroCentered
  }
  where
    i = fromIntegral :: Int -> Int32
    flag b f = if b then f else 0

-- | The config of a GGUF-loaded model: the Gemma 3 1B record with the
-- shape the file declares (vocab from token_embd's shape).
fromGh :: HIP.GhConfig -> GemmaConfig
fromGh g = gemma3_1BConfig
  { gcVocabSize = n HIP.ghVocab, gcHiddenDim = n HIP.ghHidden, gcNumLayers = n HIP.ghLayers
  , gcNumHeads = n HIP.ghHeads, gcNumKVHeads = n HIP.ghKVHeads, gcHeadDim = n HIP.ghHeadDim
  , gcFFNDim = n HIP.ghFFN, gcRopeBase = HIP.ghThetaGlobal g
  , gcUseSlidingWindow = HIP.ghSlidingWindow g > 0, gcSlidingWindowSize = n HIP.ghSlidingWindow
  }
  where n f = fromIntegral (f g)

withModel :: HIP.Context -> HIP.Model -> GemmaConfig -> Int -> IO (GemmaModel dtype)
withModel ctx m cfg maxSeq = do
  kv <- HIP.newCache m maxSeq
  pure GemmaModel { gmConfig = cfg, gmContext = ctx, gmHandle = m, gmCache = kv, gmMaxSeq = maxSeq }

-- | loadGemmaModel (src/Gemma/Model.hs:276): SafeTensors (HF names) as f32
-- through gh_model_set_tensor under the GGUF tensor names.
loadGemmaModel :: FilePath -> GemmaConfig -> IO (GemmaModel dtype)
loadGemmaModel path cfg@GemmaConfig{..} = do
  st <- loadSafeTensors path
  ctx <- HIP.newContext 0
  m <- HIP.newModel ctx (toGh cfg defaultMaxSeq)
  let put gguf hf = do
        present <- pure (hasTensor st (T.pack hf))
        when present $ do
          v <- getTensor st (T.pack hf)
          withForeignPtr m $ \mp -> withCString gguf $ \np -> V.unsafeWith v $ \vp ->
            check (HIP.c_modelSetTensor mp np HIP.dtypeF32 (castPtr vp)
                                        (fromIntegral (V.length v * sizeOf (0 :: Float))))
  put "token_embd.weight" "model.embed_tokens.weight"
  put "output_norm.weight" "model.norm.weight"
  -- an untied LM head when the checkpoint has one; else the library uses
  -- the embedding (src/Gemma/Model.hs:412-414)
  put "output.weight" "lm_head.weight"
  forM_ [0 .. gcNumLayers - 1] $ \l -> do
    let g s = "blk." ++ show l ++ "." ++ s ++ ".weight"
        h s = "model.layers." ++ show l ++ "." ++ s ++ ".weight"
    put (g "attn_norm") (h "input_layernorm")
    put (g "attn_q") (h "self_attn.q_proj")
    put (g "attn_k") (h "self_attn.k_proj")
    put (g "attn_v") (h "self_attn.v_proj")
    put (g "attn_q_norm") (h "self_attn.q_norm")
    put (g "attn_k_norm") (h "self_attn.k_norm")
    put (g "attn_output") (h "self_attn.o_proj")
    put (g "post_attention_norm") (h "post_attention_layernorm")
    put (g "ffn_norm") (h "pre_feedforward_layernorm")
    put (g "ffn_gate") (h "mlp.gate_proj")
    put (g "ffn_up") (h "mlp.up_proj")
    put (g "ffn_down") (h "mlp.down_proj")
    put (g "post_ffw_norm") (h "post_feedforward_layernorm")
  withForeignPtr m (check . HIP.c_modelCheck)
  withModel ctx m cfg defaultMaxSeq

-- | loadGemmaModelFromGGUF (src/Gemma/Model.hs:908): the file is parsed and
-- every tensor, Q4_0 projections and the LM head included (output.weight,
-- src/Gemma/Model.hs:988, or the tied embedding), uploaded by the library
-- (gh_model_load_gguf).
loadGemmaModelFromGGUF :: FilePath -> ContT r IO (GemmaModel dtype)
loadGemmaModelFromGGUF path = liftIO $ do
  ctx <- HIP.newContext 0
  m <- HIP.loadGGUF ctx path defaultMaxSeq
  g <- withForeignPtr m $ \mp -> alloca $ \pc -> check (HIP.c_modelConfig mp pc) >> peek pc
  withModel ctx m (fromGh g) defaultMaxSeq

-- | runGemmaInference (src/Gemma/Model.hs:1248): the logits of the last
-- token of a sequence, through a batched prefill on a fresh device cache.
runGemmaInference :: GemmaModel dtype -> Vector Int -> IO (Vector Float)
runGemmaInference GemmaModel{..} tokenIds = do
  let GemmaConfig{..} = gmConfig
      toks = V.map fromIntegral tokenIds :: Vector Int32
  kv <- HIP.newCache gmHandle (max 1 (V.length tokenIds))
  logits <- VM.new gcVocabSize
  withForeignPtr gmHandle $ \m -> withForeignPtr kv $ \k -> V.unsafeWith toks $ \tp ->
    VM.unsafeWith logits $ \lp -> alloca $ \np ->
      check (HIP.c_prefill m k tp (fromIntegral (V.length toks)) (castPtr lp) nullPtr np)
  V.unsafeFreeze logits

-- | runGemmaInferenceCached (src/Gemma/Model.hs:1313-1316).
runGemmaInferenceCached :: GemmaModel dtype
                        -> Vector Int
                        -> Maybe KVCache
                        -> IO (Vector Float, KVCache)
runGemmaInferenceCached model tokenIds mCache = do
  (logits, cache, _) <- cachedStep False model tokenIds mCache
  pure (logits, cache)

-- | runGemmaInferenceCachedWithLayer0 (src/Gemma/Model.hs:1441-1444): also
-- the hidden state after layer 0.
runGemmaInferenceCachedWithLayer0 :: GemmaModel dtype
                                  -> V.Vector Int
                                  -> Maybe KVCache
                                  -> IO (V.Vector Float, KVCache, V.Vector Float)
runGemmaInferenceCachedWithLayer0 = cachedStep True

-- One decode step at the cache value's position: gh_step writes the logits
-- (and, when asked, the hidden state after every layer); the argmax it also
-- returns is what sampleToken computes from them (app/Main.hs:488-507).
cachedStep :: Bool -> GemmaModel dtype -> Vector Int -> Maybe KVCache
           -> IO (Vector Float, KVCache, Vector Float)
cachedStep wantLayers GemmaModel{..} tokenIds mCache = do
  let GemmaConfig{..} = gmConfig
      n = V.length tokenIds
  when (n /= 1) $ error ("Cached inference requires single token, got " ++ show n)
  let cache0 = fromMaybe (initKVCache gcNumLayers gcNumKVHeads gcHeadDim gmMaxSeq) mCache
      pos = cacheLength (BV.head (kvLayers cache0))
  logits <- VM.new gcVocabSize
  layers <- VM.new (if wantLayers then gcNumLayers * gcHiddenDim else 1)
  withForeignPtr gmHandle $ \m -> withForeignPtr gmCache $ \kv -> do
    check (HIP.c_kvTruncate kv (fromIntegral pos))
    VM.unsafeWith logits $ \lp -> VM.unsafeWith layers $ \yp -> alloca $ \np ->
      check (HIP.c_step m kv (fromIntegral (V.head tokenIds)) (castPtr lp)
                        (if wantLayers then castPtr yp else (nullPtr :: Ptr CFloat)) np)
  lv <- V.unsafeFreeze logits
  yv <- V.unsafeFreeze layers
  let grow l = l { cacheLen = cacheLen l + 1 }
      cache1 = KVCache { kvLayers = BV.map grow (kvLayers cache0) }
  pure (lv, cache1, if wantLayers then V.take gcHiddenDim yv else V.empty)
