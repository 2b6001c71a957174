from litevllm.entrypoints.llm import main

if __name__ == "__main__":
    main()
